// Weight-only-quant GEMV family for gfx950 (W16A16 / W8A16 / W4A16).
//
// One kernel template covers every GEMV of the decode step
// (src/kernels.cu:402-687, :772-871 in the reference):
//   * a 256-thread block stages the fp16 input vector in LDS once (optionally
//     RMS-normalising it on the way, which fuses the reference's separate
//     rmsnorm launch, kernels.cu:689-768), in a plane-major layout so that
//     every lane's 16-byte LDS read is bank-conflict free;
//   * each wave owns R weight rows and streams them with 16-byte coalesced
//     loads (one load instruction covers 1 KB of a row), unpacking int8/int4
//     in registers to fp16 pairs and accumulating with v_dot2_f32_f16 in fp32;
//   * a 64-lane butterfly reduction, then a fused epilogue (bias, residual,
//     SwiGLU, RoPE + KV-cache store, repetition penalty) writes fp16.
// No matrix cores: an M=1 GEMV is HBM-bound (0.5-2 flop/byte).
#pragma once

#include "cq_device.h"

namespace cq {

template <int Q> struct QTraits;
template <> struct QTraits<CQ_QUANT_FP16> {
  static constexpr int EPC = 8;      // logical weights per 16-byte chunk
  static constexpr int PLANES = 1;   // 16-byte x planes per chunk
  static constexpr float BIAS = 0.f;
};
template <> struct QTraits<CQ_QUANT_INT8> {
  static constexpr int EPC = 16;
  static constexpr int PLANES = 2;
  static constexpr float BIAS = kInt8Bias;
};
template <> struct QTraits<CQ_QUANT_INT4> {
  static constexpr int EPC = 32;
  static constexpr int PLANES = 4;
  static constexpr float BIAS = kInt4Bias;
};

// Sum over one 16-byte weight chunk of (unpacked weight) * x, where x holds
// the chunk's PLANES 16-byte x planes in the order the unpack produces.  For
// quantized weights the result still contains BIAS * sum(x) (removed by the
// caller once per chunk, shared by all rows).
template <int Q> __device__ __forceinline__ float chunk_dot(u4_t w, const u4_t* x);

template <> __device__ __forceinline__ float chunk_dot<CQ_QUANT_FP16>(u4_t w, const u4_t* x) {
  float a = dot2(w.x, x[0].x, 0.f);
  a = dot2(w.y, x[0].y, a);
  a = dot2(w.z, x[0].z, a);
  return dot2(w.w, x[0].w, a);
}
template <> __device__ __forceinline__ float chunk_dot<CQ_QUANT_INT8>(u4_t w, const u4_t* x) {
  // words 0,1 -> plane 0 (elements 0..7), words 2,3 -> plane 1 (8..15)
  const uint32_t f0 = w.x ^ kInt8Flip, f1 = w.y ^ kInt8Flip, f2 = w.z ^ kInt8Flip, f3 = w.w ^ kInt8Flip;
  float a = dot2(int8_pair(f0, 0), x[0].x, 0.f);
  a = dot2(int8_pair(f0, 1), x[0].y, a);
  a = dot2(int8_pair(f1, 0), x[0].z, a);
  a = dot2(int8_pair(f1, 1), x[0].w, a);
  a = dot2(int8_pair(f2, 0), x[1].x, a);
  a = dot2(int8_pair(f2, 1), x[1].y, a);
  a = dot2(int8_pair(f3, 0), x[1].z, a);
  return dot2(int8_pair(f3, 1), x[1].w, a);
}
template <> __device__ __forceinline__ float chunk_dot<CQ_QUANT_INT4>(u4_t w, const u4_t* x) {
  float a = 0.f;
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t f = words[p] ^ kInt4Flip;
    a = dot2(int4_pair(f, 0), x[p].x, a);
    a = dot2(int4_pair(f, 1), x[p].y, a);
    a = dot2(int4_pair(f, 2), x[p].z, a);
    a = dot2(int4_pair(f, 3), x[p].w, a);
  }
  return a;
}

// Order of the 8 fp16 x values of one plane as the unpack pairs them: int4
// pairs elements (0,4)(1,5)(2,6)(3,7) of each 8-weight word; int8 and fp16
// keep natural order.
template <int Q> __device__ __forceinline__ void plane_order(const float* v, _Float16* out) {
  if constexpr (Q == CQ_QUANT_INT4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = (_Float16)v[i];
      out[2 * i + 1] = (_Float16)v[i + 4];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (_Float16)v[i];
  }
}

}  // namespace cq
