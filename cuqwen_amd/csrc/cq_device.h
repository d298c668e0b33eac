// Device-side building blocks for gfx950 (wave64): vector types, the
// in-register int8/int4 -> fp16 unpack, packed fp16 dot products and wave
// reductions.
#pragma once

#include "cq_common.h"

namespace cq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t as_u32(h2_t h) { return __builtin_bit_cast(uint32_t, h); }

// v_dot2_f32_f16: a.x*b.x + a.y*b.y + c with fp32 accumulation.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// ---------------------------------------------------------------- unpack
// Int4 (export_weights.py:197-199): byte k of a 32-bit word holds element 2k
// in its low nibble and 2k+1 in its high nibble; the nibble is a 4-bit two's
// complement value q in [-8, 7] (kernels.cu:35-37 sign-extends ((n^8)-8)).
// After w ^= 0x88888888 each nibble is n = q + 8 in [0, 15].  OR-ing the
// fp16 exponent pattern 0x6400 (1024.0; fp16 spacing is 1 on [1024, 2048))
// onto a nibble left where it is gives an exact fp16:
//   (w' & 0x000F000F) | 0x64006400        -> (1024 + n0, 1024 + n4)
//   (w' & 0x00F000F0) | 0x64006400        -> (1024 + 16 n1, 1024 + 16 n5)
//   ((w' >> 8) & 0x000F000F) | 0x64006400 -> (1024 + n2, 1024 + n6)
//   ((w' >> 8) & 0x00F000F0) | 0x64006400 -> (1024 + 16 n3, 1024 + 16 n7)
// The staged x plane pairs each with (x0, x4), (x1/16, x5/16), (x2, x6),
// (x3/16, x7/16), so that (1024 + n) x = q x + 1032 x and
// (1024 + 16 n) x / 16 = q x + 72 x: one shift, four and-or and four dot2 per
// eight weights; the 1032 / 72 terms are removed once per chunk.
constexpr uint32_t kInt4Flip = 0x88888888u;
constexpr float kInt4BiasLo = 1032.0f;
constexpr float kInt4BiasHi = 72.0f;
// Int8: byte b of a word is q in [-128, 127]; u = q ^ 0x80 = q + 128 and the
// fp16 with bits 0x64uu is 1024 + u = 1152 + q.  v_perm_b32 builds the pair
// (byte 2i, byte 2i+1) with 0x64 high bytes in one instruction.
constexpr uint32_t kInt8Flip = 0x80808080u;
constexpr float kInt8Bias = 1152.0f;

// A constant held in a VGPR: gfx9 VOP3 instructions read at most one scalar
// operand, so v_and_or_b32 / v_perm_b32 with two constants would otherwise
// be split into two instructions.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
  uint32_t v;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "s"(c));
  return v;
}
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask_v, uint32_t c) { return (a & mask_v) | c; }

__device__ __forceinline__ uint32_t int8_pair(uint32_t flipped, uint32_t magic_v, int i) {
  // selector bytes 0-3 pick bytes of src1 (flipped), 4-7 bytes of src0.
  return __builtin_amdgcn_perm(magic_v, flipped, i == 0 ? 0x04010400u : 0x04030402u);
}

// ------------------------------------------------------------- reductions
// Wave-wide reductions on DPP lane moves: four in-row steps (quad swaps,
// half-row and row mirrors) leave every lane of a 16-lane row holding the
// row's result, then the four row results are combined through scalar
// registers.  Every lane ends with the bitwise-identical value (each step
// combines the same two operands on both lanes of a pair), and nothing goes
// through LDS, unlike a shuffle (ds_bpermute) butterfly.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_of(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
constexpr int kDppQuadSwap1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<kDppQuadSwap1>(v);
  v += dpp_mov<kDppQuadSwap2>(v);
  v += dpp_mov<kDppRowHalfMirror>(v);
  v += dpp_mov<kDppRowMirror>(v);
  return (lane_of(v, 0) + lane_of(v, 16)) + (lane_of(v, 32) + lane_of(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp_mov<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp_mov<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_mov<kDppRowMirror>(v));
  return fmaxf(fmaxf(lane_of(v, 0), lane_of(v, 16)), fmaxf(lane_of(v, 32), lane_of(v, 48)));
}

// NeoX RoPE rotation of one pair (y0, y1) = (v[i], v[i + hd/2])
// (kernels.cu:370-398): the angle pos * inv_freq (inv_freq = theta^(-2i/hd)
// in double) is reduced modulo 2 pi in double (2 pi split in a high and a
// low part) and its sine and cosine taken in fp32; the rotation is rounded
// at the same points as the reference's fp32 expression.
// RoPE inverse frequency theta^(-2i/hd) in double, for callers without the
// host-computed table (the op-level entry points).
__device__ __forceinline__ double rope_inv_freq_dev(float theta, int i, int hd) {
  return 1.0 / pow((double)theta, (2.0 * i) / (double)hd);
}
__device__ __forceinline__ void rope_sincos(int pos, double inv_freq, float* s, float* c) {
  const double ang = (double)pos * inv_freq;
  const double k = rint(ang * 0.15915494309189535);                                        // 1 / (2 pi)
  const double rd = fma(-k, 6.283185307179586232e+00, ang) - k * 2.4492935982947064e-16;   // 2 pi hi + lo
  sincosf((float)rd, s, c);
}
__device__ __forceinline__ void rope_apply(float& y0, float& y1, float s, float c) {
  const float o0 = add_rn(mul_rn(y0, c), -mul_rn(y1, s));
  const float o1 = add_rn(mul_rn(y1, c), mul_rn(y0, s));
  y0 = o0;
  y1 = o1;
}
__device__ __forceinline__ void rope_rotate(float& y0, float& y1, int pos, double inv_freq) {
  float s, c;
  rope_sincos(pos, inv_freq, &s, &c);
  rope_apply(y0, y1, s, c);
}

// Order-preserving argmax key (kernels.cu:907-911): a larger float gives a
// larger key, equal floats let the lower index win (~idx), NaN sorts above
// +inf.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  const uint32_t fu = __float_as_uint(v);
  const uint32_t key = (fu & 0x80000000u) ? ~fu : (fu | 0x80000000u);
  return ((unsigned long long)key << 32) | (uint32_t)(~idx);
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off, kWave);
    v = o > v ? o : v;
  }
  return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024); `red` holds 16
// floats of LDS.  All threads get the result.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave, nw = blockDim.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// s_barrier that is also a compiler memory barrier: no LDS or global access
// is moved across it (a bare __builtin_amdgcn_s_barrier is not one), while
// no wait is added -- the caller waits for its own LDS stores (lgkmcnt)
// first, and the weight loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// A 32-bit word that no wave of the running kernel writes (a control word
// written by an earlier launch or the host), read through the constant
// address space: the compiler issues a scalar load, whose wait counts only
// scalar loads.  As a vector load from a uniform address it was turned into
// a scalar with readfirstlane right away, behind a full vmcnt(0) that waited
// for every load the wave had in flight.  (The scalar cache is invalidated
// at each kernel launch, so earlier writes are seen.)
__device__ __forceinline__ uint32_t load_ctl_u32(const void* p) {
  return *(const __attribute__((address_space(4))) uint32_t*)p;
}

__device__ __forceinline__ u4_t load_u4(const void* p) { return *reinterpret_cast<const u4_t*>(p); }

// Makes the compiler materialise a kernel-argument value in an SGPR here.
// Pinning every argument a kernel reads at its entry puts all their scalar
// loads in one batch with one wait; otherwise each is loaded where first
// used and a prologue waits for several dependent kernel-argument round
// trips (≈0.35 us each) before its first streaming load.
#define CQ_PIN(v) asm volatile("" ::"s"(v))
// Buffer resource over `base` (word 3: the gfx9 32-bit data format), of
// 2^31 - 1 bytes when `valid`, else of none: a load through the empty one
// returns zeros at once without a memory request.  Lets a loop issue the
// same loads on every path (exact wait counts) while steps past its range
// cost nothing.
constexpr int kBufWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_or_null(const void* base, bool valid) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, valid ? 0x7fffffff : 0, kBufWord3);
}
constexpr int kCacheNT = 2;   // buffer load cache policy: non-temporal (streamed once)

__device__ __forceinline__ u4_t load_u4_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p));
}

}  // namespace cq
