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
};
template <> struct QTraits<CQ_QUANT_INT8> {
  static constexpr int EPC = 16;
  static constexpr int PLANES = 2;
};
template <> struct QTraits<CQ_QUANT_INT4> {
  static constexpr int EPC = 32;
  static constexpr int PLANES = 4;
};

// Constants of the unpack kept in VGPRs for the whole kernel.
struct UnpackRegs {
  uint32_t m_lo, m_hi, magic;
};
__device__ __forceinline__ UnpackRegs unpack_regs() {
  return UnpackRegs{vgpr_const(0x000F000Fu), vgpr_const(0x00F000F0u), vgpr_const(0x64646464u)};
}

// Sum over one 16-byte weight chunk of (unpacked weight) * x, where x holds
// the chunk's PLANES 16-byte x planes in the order the unpack produces.  For
// quantized weights the result still contains the unpack bias times the
// chunk's x (removed by the caller once per chunk, shared by all rows).
template <int Q> __device__ __forceinline__ float chunk_dot(u4_t w, const u4_t* x, const UnpackRegs& k);

template <> __device__ __forceinline__ float chunk_dot<CQ_QUANT_FP16>(u4_t w, const u4_t* x, const UnpackRegs&) {
  float a = dot2(w.x, x[0].x, 0.f);
  float b = dot2(w.y, x[0].y, 0.f);
  a = dot2(w.z, x[0].z, a);
  b = dot2(w.w, x[0].w, b);
  return a + b;
}
template <> __device__ __forceinline__ float chunk_dot<CQ_QUANT_INT8>(u4_t w, const u4_t* x, const UnpackRegs& k) {
  // words 0,1 -> plane 0 (elements 0..7), words 2,3 -> plane 1 (8..15)
  const uint32_t f0 = w.x ^ kInt8Flip, f1 = w.y ^ kInt8Flip, f2 = w.z ^ kInt8Flip, f3 = w.w ^ kInt8Flip;
  float a = dot2(int8_pair(f0, k.magic, 0), x[0].x, 0.f);
  float b = dot2(int8_pair(f0, k.magic, 1), x[0].y, 0.f);
  a = dot2(int8_pair(f1, k.magic, 0), x[0].z, a);
  b = dot2(int8_pair(f1, k.magic, 1), x[0].w, b);
  a = dot2(int8_pair(f2, k.magic, 0), x[1].x, a);
  b = dot2(int8_pair(f2, k.magic, 1), x[1].y, b);
  a = dot2(int8_pair(f3, k.magic, 0), x[1].z, a);
  b = dot2(int8_pair(f3, k.magic, 1), x[1].w, b);
  return a + b;
}
template <> __device__ __forceinline__ float chunk_dot<CQ_QUANT_INT4>(u4_t w, const u4_t* x, const UnpackRegs& k) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t f = words[p] ^ kInt4Flip;
    const uint32_t f8 = f >> 8;
    float& a = acc[p & 1];
    a = dot2(and_or(f, k.m_lo, 0x64006400u), x[p].x, a);
    a = dot2(and_or(f, k.m_hi, 0x64006400u), x[p].y, a);
    a = dot2(and_or(f8, k.m_lo, 0x64006400u), x[p].z, a);
    a = dot2(and_or(f8, k.m_hi, 0x64006400u), x[p].w, a);
  }
  return acc[0] + acc[1];
}

// Order of the 8 fp16 x values of one plane as the unpack pairs them, and
// the plane's unpack-bias term: int4 pairs (0,4) (1/16,5/16) (2,6)
// (3/16,7/16) and owes 1032 * (x0+x4+x2+x6) + 72 * (x1+x5+x3+x7); int8 keeps
// natural order and owes 1152 * sum(x); fp16 owes nothing.
template <int Q> __device__ __forceinline__ float plane_order(const float* v, _Float16* out) {
  if constexpr (Q == CQ_QUANT_INT4) {
    out[0] = (_Float16)v[0]; out[1] = (_Float16)v[4];
    out[2] = (_Float16)(v[1] * 0.0625f); out[3] = (_Float16)(v[5] * 0.0625f);
    out[4] = (_Float16)v[2]; out[5] = (_Float16)v[6];
    out[6] = (_Float16)(v[3] * 0.0625f); out[7] = (_Float16)(v[7] * 0.0625f);
    return kInt4BiasLo * (v[0] + v[4] + v[2] + v[6]) + kInt4BiasHi * (v[1] + v[5] + v[3] + v[7]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (_Float16)v[i];
    if constexpr (Q == CQ_QUANT_INT8) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s += v[i];
      return kInt8Bias * s;
    }
    return 0.f;
  }
}

}  // namespace cq
