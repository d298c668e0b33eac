// Weight-file format (export_weights.py:267-323) and the synthetic weight
// generator: host side.
#pragma once

#include "cq_common.h"

#include <vector>

namespace cq {

// One tensor of the file, in file order.
struct TensorSpec {
  int kind;        // TensorKind
  int layer;       // -1 for global tensors
  int64_t rows;    // 1 for vectors
  int64_t cols;
  int quant;       // storage: CQ_QUANT_FP16 / INT8 / INT4
  int64_t weight_bytes;
  int64_t scale_bytes;   // 0 for fp16 tensors
};

int validate_config(const cq_config& c);
std::vector<TensorSpec> tensor_list(const cq_config& c);
int64_t file_bytes(const cq_config& c);

// Generator constants of one tensor kind.
float kind_mean(int kind);

// Quantize [rows][cols] fp16 to int8/int4 with group `group` (export_weights.py:123-205).
void quantize_host(int quant, const uint16_t* w, int64_t rows, int64_t cols, int group, uint8_t* q, uint16_t* s);

// Host generation of one tensor (fp16 values before quantization).
void synth_tensor_host(uint64_t seed, const TensorSpec& t, std::vector<uint16_t>& out);

}  // namespace cq
