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

// Staging transform of one 16-byte plane of the input (8 fp16 values m0..m7,
// already x or half(x * w)) into the order the unpack pairs it, plus the
// plane's unpack-bias term: int4 pairs (m0,m4) (m1/16,m5/16) (m2,m6)
// (m3/16,m7/16) and owes 1032 * (m0+m4+m2+m6) + 72 * (m1+m5+m3+m7); int8
// keeps natural order and owes 1152 * sum(m); fp16 owes nothing.  Packed
// fp16 arithmetic throughout (m/16 is the correctly rounded quotient); the
// bias term is summed in fp32 with dot2 instructions.
template <int Q> __device__ __forceinline__ float plane_order_packed(const u4_t& m, u4_t& out) {
  if constexpr (Q == CQ_QUANT_INT4) {
    const h2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2_t blo = {(_Float16)kInt4BiasLo, (_Float16)kInt4BiasLo};
    const h2_t bhi = {(_Float16)kInt4BiasHi, (_Float16)kInt4BiasHi};
    const uint32_t p04 = __builtin_amdgcn_perm(m.z, m.x, 0x05040100u);   // (m0, m4)
    const uint32_t p15 = __builtin_amdgcn_perm(m.z, m.x, 0x07060302u);   // (m1, m5)
    const uint32_t p26 = __builtin_amdgcn_perm(m.w, m.y, 0x05040100u);   // (m2, m6)
    const uint32_t p37 = __builtin_amdgcn_perm(m.w, m.y, 0x07060302u);   // (m3, m7)
    out.x = p04;
    out.y = as_u32(as_h2(p15) * sixteenth);
    out.z = p26;
    out.w = as_u32(as_h2(p37) * sixteenth);
    float c = __builtin_amdgcn_fdot2(as_h2(p04), blo, 0.f, false);
    c = __builtin_amdgcn_fdot2(as_h2(p26), blo, c, false);
    c = __builtin_amdgcn_fdot2(as_h2(p15), bhi, c, false);
    return __builtin_amdgcn_fdot2(as_h2(p37), bhi, c, false);
  } else {
    out = m;
    if constexpr (Q == CQ_QUANT_INT8) {
      const h2_t b8 = {(_Float16)kInt8Bias, (_Float16)kInt8Bias};
      float c = __builtin_amdgcn_fdot2(as_h2(m.x), b8, 0.f, false);
      c = __builtin_amdgcn_fdot2(as_h2(m.y), b8, c, false);
      c = __builtin_amdgcn_fdot2(as_h2(m.z), b8, c, false);
      return __builtin_amdgcn_fdot2(as_h2(m.w), b8, c, false);
    }
    return 0.f;
  }
}

}  // namespace cq
