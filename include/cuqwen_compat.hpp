// cuqwen_compat.hpp -- the reference's C++ decode API over the C ABI of
// cuqwen.h, for callers written against talhatahir-10xe/CuQwen:
//
//   struct QwenConfig                       include/config.h:52-127
//   struct LayerWeights / QwenWeights       include/load_weights.h:17-54
//   load_weights / free_weights             include/load_weights.h:57-60
//   struct QwenState                        include/model.cuh:9-46
//   malloc_qwen_state / free_qwen_state     include/model.cuh:48-49
//   qwen_forward                            include/model.cuh:51-60
//   launch_embedding_lookup                 include/kernels.cuh:19
//   launch_gqa_attention_decode             include/kernels.cuh:21-35
//   launch_kv_cache_store                   include/kernels.cuh:37-47
//   launch_apply_repetition_penalty         include/kernels.cuh:49-56
//   launch_argmax                           include/kernels.cuh:58-63
//   launch_fused_attn_block                 include/kernels.cuh:69-94
//   launch_fused_mlp_stage1 / _stage2       include/kernels.cuh:96-120
//   launch_gemv_add_fp16                    include/kernels.cuh:122-130
//   launch_rmsnorm                          include/kernels.cuh:132-139
//   launch_compute_logits / _int8           include/kernels.cuh:141-160
//
// Model and precision are chosen at compile time with the reference's own
// macros (-DQWEN_MODEL_0_5B | _1_5B | _3B | _7B | _14B, and -DQUANT_INT8 or
// -DQUANT_INT4 for a quantized build; fp16 otherwise), so a caller keeps
// QwenConfig::model_name, QwenConfig::bin_path, QwenConfig::max_seq_len and
// config.vocab_size as it uses them.  Header only; link with -lcuqwen.
//
// What differs from the reference: errors throw std::runtime_error (with
// cq_last_error()'s message) instead of exit(EXIT_FAILURE); the stream
// argument is a hipStream_t; QwenState's members are the engine's (a handle
// to its state), not the reference's buffers.
#ifndef CUQWEN_COMPAT_HPP
#define CUQWEN_COMPAT_HPP

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "cuqwen.h"

constexpr int QUANT_GROUP_SIZE = CQ_QUANT_GROUP;
// Split-K partial buffers of launch_gqa_attention_decode, sized as the
// reference sizes them (include/kernels.cuh:17, include/config.h:146).
constexpr int PARTIAL_HEAD_SLOTS = 16;
constexpr int ATTN_PARTITIONS = 64;

// include/config.h:18-40: weight element type, row stride in qweight_t
// elements, QUANT_ENABLED for the builds with scales
#if defined(QUANT_INT8)
using qweight_t = int8_t;
#define CQ_COMPAT_QUANT_TAG "int8"
#define CQ_COMPAT_QUANT CQ_QUANT_INT8
#define QUANT_ENABLED
#define WEIGHT_ROW_STRIDE(cols) (cols)
#elif defined(QUANT_INT4)
using qweight_t = int8_t;   // two 4-bit weights per byte
#define CQ_COMPAT_QUANT_TAG "int4"
#define CQ_COMPAT_QUANT CQ_QUANT_INT4
#define QUANT_ENABLED
#define WEIGHT_ROW_STRIDE(cols) ((cols) / 2)
#else
#define WEIGHT_ROW_STRIDE(cols) (cols)
using qweight_t = __half;
#define CQ_COMPAT_QUANT_TAG "fp16"
#define CQ_COMPAT_QUANT CQ_QUANT_FP16
#endif

// The five presets (model values of include/config.h:55-113).
#if defined(QWEN_MODEL_0_5B)
#define CQ_COMPAT_MODEL "0.5B", "0_5b", 151936, 896, 4864, 24, 14, 2, 64
#elif defined(QWEN_MODEL_1_5B)
#define CQ_COMPAT_MODEL "1.5B", "1_5b", 151936, 1536, 8960, 28, 12, 2, 128
#elif defined(QWEN_MODEL_3B)
#define CQ_COMPAT_MODEL "3B", "3b", 151936, 2048, 11008, 36, 16, 2, 128
#elif defined(QWEN_MODEL_7B)
#define CQ_COMPAT_MODEL "7B", "7b", 152064, 3584, 18944, 28, 28, 4, 128
#elif defined(QWEN_MODEL_14B)
#define CQ_COMPAT_MODEL "14B", "14b", 152064, 5120, 13824, 48, 40, 8, 128
#else
#error "define one of QWEN_MODEL_0_5B, QWEN_MODEL_1_5B, QWEN_MODEL_3B, QWEN_MODEL_7B, QWEN_MODEL_14B"
#endif

namespace cq_compat {
struct Preset {
  const char* name;
  const char* tag;
  int32_t vocab, dim, inter, layers, heads, kv_heads, head_dim;
};
constexpr Preset kPreset{CQ_COMPAT_MODEL};
constexpr const char* kBinPath[5][3] = {
    {"weights/model_fp16_0_5b.bin", "weights/model_int8_0_5b.bin", "weights/model_int4_0_5b.bin"},
    {"weights/model_fp16_1_5b.bin", "weights/model_int8_1_5b.bin", "weights/model_int4_1_5b.bin"},
    {"weights/model_fp16_3b.bin", "weights/model_int8_3b.bin", "weights/model_int4_3b.bin"},
    {"weights/model_fp16_7b.bin", "weights/model_int8_7b.bin", "weights/model_int4_7b.bin"},
    {"weights/model_fp16_14b.bin", "weights/model_int8_14b.bin", "weights/model_int4_14b.bin"}};
constexpr int model_index(const char* tag) {
  return tag[0] == '0' ? 0 : tag[0] == '3' ? 2 : tag[0] == '7' ? 3 : tag[1] == '_' ? 1 : 4;
}

[[noreturn]] inline void raise(const char* what) {
  throw std::runtime_error(std::string(what) + ": " + cq_last_error());
}
inline void check(int rc, const char* what) {
  if (rc != CQ_OK) raise(what);
}
}  // namespace cq_compat

struct QwenConfig {
  static constexpr int32_t magic = CQ_MAGIC;
  static constexpr const char* model_name = cq_compat::kPreset.name;
  static constexpr int32_t vocab_size = cq_compat::kPreset.vocab;
  static constexpr int32_t dim = cq_compat::kPreset.dim;
  static constexpr int32_t intermediate_size = cq_compat::kPreset.inter;
  static constexpr int32_t n_layers = cq_compat::kPreset.layers;
  static constexpr int32_t n_heads = cq_compat::kPreset.heads;
  static constexpr int32_t n_kv_heads = cq_compat::kPreset.kv_heads;
  static constexpr int32_t head_dim = cq_compat::kPreset.head_dim;
  static constexpr int32_t max_seq_len = 32768;
  static constexpr const char* bin_path =
      cq_compat::kBinPath[cq_compat::model_index(cq_compat::kPreset.tag)][CQ_COMPAT_QUANT];
  static constexpr int32_t quant_type = CQ_COMPAT_QUANT;
  static constexpr float norm_eps = 1e-6f;
  static constexpr float rope_theta = 1000000.0f;
  static constexpr float repetition_penalty = 1.1f;

  // The engine's run-time config of this build (preset + exporter lm_head rule).
  static cq_config runtime() {
    cq_config c{};
    cq_compat::check(cq_config_preset(model_name, quant_type, &c), "QwenConfig");
    return c;
  }
};

// Device pointers into the engine's weights, filled by load_weights so
// op-level callers find every tensor where the reference's loader puts it,
// all in the exporter's layout.  o_proj_weight / o_proj_scale point at a
// row-major copy (cq_weights_wo_rows): the engine's own Wo is held in
// 128-column panels for its merged O-projection, and a caller that runs
// launch_gemv_add_fp16 on these pointers (src/model.cu:129) gets the
// reference's result.
struct LayerWeights {
  __half* input_layernorm_weight = nullptr;
  qweight_t* q_proj_weight = nullptr;
  __half* q_proj_bias = nullptr;
  qweight_t* k_proj_weight = nullptr;
  __half* k_proj_bias = nullptr;
  qweight_t* v_proj_weight = nullptr;
  __half* v_proj_bias = nullptr;
  qweight_t* o_proj_weight = nullptr;
  __half* post_attention_layernorm_weight = nullptr;
  qweight_t* gate_proj_weight = nullptr;
  qweight_t* up_proj_weight = nullptr;
  qweight_t* down_proj_weight = nullptr;
  __half* q_proj_scale = nullptr;
  __half* k_proj_scale = nullptr;
  __half* v_proj_scale = nullptr;
  __half* o_proj_scale = nullptr;
  __half* gate_proj_scale = nullptr;
  __half* up_proj_scale = nullptr;
  __half* down_proj_scale = nullptr;
};

struct QwenWeights {
  __half* embed_tokens = nullptr;
  std::vector<LayerWeights> layers;
  __half* norm_weight = nullptr;
  __half* lm_head_weight = nullptr;   // fp16 head, or embed_tokens when tied
  bool lm_head_quantized = false;
  int8_t* lm_head_q = nullptr;
  __half* lm_head_scale = nullptr;
  cq_weights* handle = nullptr;       // the engine's weights
};

struct QwenState {
  cq_state* handle = nullptr;
};

namespace cq_compat {
template <class T>
inline T* tensor(cq_weights* w, const char* name, int layer) {
  void* p = nullptr;
  size_t bytes = 0;
  if (cq_weights_tensor(w, name, layer, &p, &bytes) != CQ_OK) return nullptr;   // absent (e.g. fp16 scales)
  return static_cast<T*>(p);
}
}  // namespace cq_compat

// load_weights (include/load_weights.h:57): the file must match this build's
// model and precision, as the reference checks against its QwenConfig.
inline QwenConfig load_weights(const std::string& bin_path, QwenWeights& w) {
  using namespace cq_compat;
  const cq_config expect = QwenConfig::runtime();
  cq_config got{};
  check(cq_load_weights(bin_path.c_str(), &expect, &got, &w.handle), "load_weights");
  w.embed_tokens = tensor<__half>(w.handle, "embed", -1);
  w.norm_weight = tensor<__half>(w.handle, "final_norm", -1);
  w.lm_head_quantized = got.lm_head_fmt == CQ_LMHEAD_INT8;
  if (w.lm_head_quantized) {
    w.lm_head_q = tensor<int8_t>(w.handle, "lm_head", -1);
    w.lm_head_scale = tensor<__half>(w.handle, "lm_head_scale", -1);
  } else {
    w.lm_head_weight = tensor<__half>(w.handle, "lm_head", -1);
  }
  w.layers.assign(got.n_layers, LayerWeights{});
  for (int l = 0; l < got.n_layers; ++l) {
    LayerWeights& L = w.layers[l];
    L.input_layernorm_weight = tensor<__half>(w.handle, "in_norm", l);
    L.q_proj_weight = tensor<qweight_t>(w.handle, "wq", l);
    L.q_proj_bias = tensor<__half>(w.handle, "bq", l);
    L.k_proj_weight = tensor<qweight_t>(w.handle, "wk", l);
    L.k_proj_bias = tensor<__half>(w.handle, "bk", l);
    L.v_proj_weight = tensor<qweight_t>(w.handle, "wv", l);
    L.v_proj_bias = tensor<__half>(w.handle, "bv", l);
    void* wo = nullptr;
    void* so = nullptr;
    check(cq_weights_wo_rows(w.handle, l, &wo, &so), "load_weights (o_proj rows)");
    L.o_proj_weight = static_cast<qweight_t*>(wo);
    L.o_proj_scale = static_cast<__half*>(so);
    L.post_attention_layernorm_weight = tensor<__half>(w.handle, "post_norm", l);
    L.gate_proj_weight = tensor<qweight_t>(w.handle, "wg", l);
    L.up_proj_weight = tensor<qweight_t>(w.handle, "wu", l);
    L.down_proj_weight = tensor<qweight_t>(w.handle, "wd", l);
    L.q_proj_scale = tensor<__half>(w.handle, "sq", l);
    L.k_proj_scale = tensor<__half>(w.handle, "sk", l);
    L.v_proj_scale = tensor<__half>(w.handle, "sv", l);
    L.gate_proj_scale = tensor<__half>(w.handle, "sg", l);
    L.up_proj_scale = tensor<__half>(w.handle, "su", l);
    L.down_proj_scale = tensor<__half>(w.handle, "sd", l);
  }
  return QwenConfig{};
}

// free_weights (include/load_weights.h:60).
inline void free_weights(QwenWeights& w, const QwenConfig&) {
  cq_free_weights(w.handle);
  w = QwenWeights{};
}

// malloc_qwen_state (include/model.cuh:48): state for this build's config,
// KV cache zeroed; the weights are bound by the first qwen_forward.
inline void malloc_qwen_state(const QwenConfig&, QwenState& s) {
  const cq_config c = QwenConfig::runtime();
  cq_compat::check(cq_state_create(&c, nullptr, &s.handle), "malloc_qwen_state");
}

// free_qwen_state (include/model.cuh:49).
inline void free_qwen_state(QwenState& s) {
  cq_state_destroy(s.handle);
  s.handle = nullptr;
}

// qwen_forward (include/model.cuh:51-60): one synchronous decode step on
// `stream` (the state's own stream when 0); returns the greedy id after the
// repetition penalty over h_history[0..history_len).
inline int qwen_forward(int token, int pos, const QwenConfig&, QwenState& s, const QwenWeights& w,
                        const int* h_history = nullptr, int history_len = 0, hipStream_t stream = 0) {
  int32_t next = -1;
  cq_compat::check(cq_forward_ex(s.handle, w.handle, token, pos, h_history, history_len,
                                 static_cast<void*>(stream), &next),
                   "qwen_forward");
  return next;
}

// ------------------------------------------------------------------ op level
// The reference's launch_* family (include/kernels.cuh:19-160) with its
// signatures: qweight_t weights of this build's precision (-DQUANT_*),
// row-major as the exporter writes them, scales NULL for fp16; `half eps` /
// `half penalty` as the reference passes them.  Asynchronous on `stream`;
// a rejected argument throws std::runtime_error.

namespace cq_compat {
inline void* as_stream(hipStream_t s) { return static_cast<void*>(s); }

// Device workspace behind launch_argmax / launch_apply_repetition_penalty,
// which take none in the reference's signatures (it holds a function-local
// static too, src/kernels.cu:953): allocated on first use, zeroed, grown when
// a larger vocabulary needs more, kept until the process ends.  Like the
// reference's, not safe for concurrent callers.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  void* get(size_t need) {
    if (need > bytes) {
      if (ptr && hipFree(ptr) != hipSuccess) throw std::runtime_error("cuqwen_compat: hipFree failed");
      ptr = nullptr;
      bytes = 0;
      if (hipMalloc(&ptr, need) != hipSuccess || hipMemset(ptr, 0, need) != hipSuccess)
        throw std::runtime_error("cuqwen_compat: workspace allocation failed");
      bytes = need;
    }
    return ptr;
  }
};
inline Workspace& argmax_ws() {
  static Workspace w;
  return w;
}
inline Workspace& penalty_ws() {
  static Workspace w;
  return w;
}
}  // namespace cq_compat

inline void launch_embedding_lookup(const __half* embed_table, const int* d_token_id, __half* output, int dim,
                                    hipStream_t stream = 0) {
  cq_compat::check(cq_embedding_lookup(embed_table, d_token_id, output, dim, cq_compat::as_stream(stream)),
                   "launch_embedding_lookup");
}

inline void launch_apply_repetition_penalty(__half* logits, const int* d_history, const int* d_history_len,
                                            int vocab_size, __half penalty, hipStream_t stream = 0) {
  void* ws = cq_compat::penalty_ws().get(cq_penalty_workspace_bytes(vocab_size));
  cq_compat::check(cq_apply_repetition_penalty(logits, d_history, d_history_len, vocab_size, __half2float(penalty), ws,
                                               cq_compat::as_stream(stream)),
                   "launch_apply_repetition_penalty");
}

inline void launch_argmax(const __half* logits, int* d_sampled_token, int vocab_size, hipStream_t stream = 0) {
  void* ws = cq_compat::argmax_ws().get(cq_argmax_workspace_bytes(vocab_size));
  cq_compat::check(cq_argmax(logits, d_sampled_token, vocab_size, ws, cq_compat::as_stream(stream)), "launch_argmax");
}

// x is already RMS-normalized: the reference leaves norm_weight and eps
// unused (src/kernels.cu:502), and so does this wrapper.
inline void launch_fused_attn_block(const __half* x, const __half* norm_weight, const qweight_t* W_q,
                                    const qweight_t* W_k, const qweight_t* W_v, const __half* W_q_scale,
                                    const __half* W_k_scale, const __half* W_v_scale, const __half* b_q,
                                    const __half* b_k, const __half* b_v, __half* q_out, __half* k_out,
                                    __half* v_out, int dim, int q_dim, int kv_dim, int n_heads, int n_kv_heads,
                                    int head_dim, const int* d_pos, float rope_theta, __half eps,
                                    hipStream_t stream = 0) {
  (void)norm_weight;
  (void)eps;
  if (q_dim != n_heads * head_dim || kv_dim != n_kv_heads * head_dim)
    throw std::runtime_error("launch_fused_attn_block: q_dim / kv_dim do not match the head counts");
  cq_compat::check(cq_fused_attn_block(CQ_COMPAT_QUANT, x, nullptr, W_q, W_k, W_v, W_q_scale, W_k_scale, W_v_scale,
                                       b_q, b_k, b_v, q_out, k_out, v_out, dim, n_heads, n_kv_heads, head_dim, d_pos,
                                       rope_theta, 0.f, cq_compat::as_stream(stream)),
                   "launch_fused_attn_block");
}

// x is already RMS-normalized (src/kernels.cu:576).
inline void launch_fused_mlp_stage1(const __half* x, const __half* norm_weight, const qweight_t* gate_weight,
                                    const qweight_t* up_weight, const __half* gate_scale, const __half* up_scale,
                                    __half* intermediate_out, int dim, int inter_dim, __half eps,
                                    hipStream_t stream = 0) {
  (void)norm_weight;
  (void)eps;
  cq_compat::check(cq_fused_mlp_stage1(CQ_COMPAT_QUANT, x, nullptr, gate_weight, up_weight, gate_scale, up_scale,
                                       intermediate_out, dim, inter_dim, 0.f, cq_compat::as_stream(stream)),
                   "launch_fused_mlp_stage1");
}

inline void launch_fused_mlp_stage2(__half* x, const qweight_t* down_weight, const __half* down_scale,
                                    const __half* intermediate_in, int dim, int inter_dim, hipStream_t stream = 0) {
  cq_compat::check(cq_fused_mlp_stage2(CQ_COMPAT_QUANT, x, down_weight, down_scale, intermediate_in, dim, inter_dim,
                                       cq_compat::as_stream(stream)),
                   "launch_fused_mlp_stage2");
}

inline void launch_gemv_add_fp16(const qweight_t* W, const __half* W_scale, const __half* input, __half* x_inout,
                                 int rows, int cols, hipStream_t stream = 0) {
  cq_compat::check(cq_gemv_add(CQ_COMPAT_QUANT, W, W_scale, input, x_inout, rows, cols, cq_compat::as_stream(stream)),
                   "launch_gemv_add_fp16");
}

inline void launch_rmsnorm(const __half* x, const __half* norm_weight, __half* out, int dim, __half eps,
                           hipStream_t stream = 0) {
  cq_compat::check(cq_rmsnorm(x, norm_weight, out, dim, __half2float(eps), cq_compat::as_stream(stream)),
                   "launch_rmsnorm");
}

inline void launch_compute_logits(const __half* x_normed, const __half* lm_head_weight, __half* logits,
                                  int vocab_size, int dim, hipStream_t stream = 0) {
  cq_compat::check(cq_compute_logits(CQ_LMHEAD_FP16, x_normed, lm_head_weight, nullptr, logits, vocab_size, dim,
                                     cq_compat::as_stream(stream)),
                   "launch_compute_logits");
}

inline void launch_compute_logits_int8(const __half* x_normed, const int8_t* lm_head_w, const __half* lm_head_scale,
                                       __half* logits, int vocab_size, int dim, hipStream_t stream = 0) {
  cq_compat::check(cq_compute_logits(CQ_LMHEAD_INT8, x_normed, lm_head_w, lm_head_scale, logits, vocab_size, dim,
                                     cq_compat::as_stream(stream)),
                   "launch_compute_logits_int8");
}

// Op level over the reference's head-major cache (include/kernels.cuh:21-47).
inline void launch_gqa_attention_decode(const __half* q, const __half* key_cache, const __half* value_cache,
                                        __half* attn_out, const int* d_pos, int n_heads, int n_kv_heads, int head_dim,
                                        int max_seq_len, float* d_partial_out, float* d_partial_max,
                                        float* d_partial_sum, hipStream_t stream = 0) {
  cq_compat::check(cq_gqa_attention_decode_hm(q, key_cache, value_cache, attn_out, d_pos, n_heads, n_kv_heads,
                                              head_dim, max_seq_len, d_partial_out, d_partial_max, d_partial_sum,
                                              static_cast<void*>(stream)),
                   "launch_gqa_attention_decode");
}

inline void launch_kv_cache_store(const __half* k_src, const __half* v_src, __half* layer_k_cache,
                                  __half* layer_v_cache, const int* d_pos, int n_kv_heads, int max_seq_len,
                                  int head_dim, hipStream_t stream = 0) {
  cq_compat::check(cq_kv_cache_store_hm(k_src, v_src, layer_k_cache, layer_v_cache, d_pos, n_kv_heads, max_seq_len,
                                        head_dim, static_cast<void*>(stream)),
                   "launch_kv_cache_store");
}

#endif  // CUQWEN_COMPAT_HPP
