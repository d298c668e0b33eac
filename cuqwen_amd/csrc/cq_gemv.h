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
#include "cq_internal.h"

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

// ---------------------------------------------------------------------------
// Building blocks of the GEMV kernels: input staging, weight steps, row
// mapping and epilogues.

constexpr int kNumCUs = 256;   // MI355X

template <int Q> __device__ __forceinline__ constexpr bool quantized() { return Q != CQ_QUANT_FP16; }

// x staging.  Thread t owns chunks c = t + i*BLK (i < XB) of a batch; all
// of a batch's x (and norm-weight) loads are issued at once, so the prologue
// costs one memory round trip per batch (one batch whenever the RMSNorm is
// fused: K <= kNormMaxK).  A wave whose chunks all lie past the end skips
// its loads (a wave-uniform branch); in the wave that holds the end, lanes
// past it re-read the last chunk, so the code inside stays straight-line.
// The LDS image is PLANES planes of 16-byte chunk slices (bank-conflict-free
// 16-byte reads in the main loop) plus the per-chunk unpack-bias term.
//
// Fused RMSNorm (kernels.cu:689-751): the staged vector is half(x * w) and
// the scalar rsqrt(mean(x^2) + eps) multiplies each finished row sum, so the
// block reduction of x^2 rides on the staging barrier instead of adding a
// dependent step before the weights can be consumed.  (The reference rounds
// x * inv * w to fp16; here x * w is rounded and inv applied in fp32.)
constexpr int kNormMaxK = 16384;

template <int Q, bool NORM, int BLK>
struct XStage {
  static constexpr int P = QTraits<Q>::PLANES;
  // chunk slots per thread in one batch: all of x with the norm fused; without
  // it at least 512 chunks per batch (a 256-thread block would otherwise
  // stage the 304 chunks of the K=4864 int8 GEMV in two dependent round trips)
  static constexpr int XB = NORM ? (kNormMaxK / QTraits<Q>::EPC + BLK - 1) / BLK : (BLK < 512 ? 512 / BLK : 1);
  u4_t x[XB][P];
  u4_t w[NORM ? XB : 1][P];
};

// first chunk of slot i of `batch` for the calling wave (wave-uniform)
template <int Q, bool NORM, int BLK>
__device__ __forceinline__ int stage_base(int batch, int i) {
  return (batch * XStage<Q, NORM, BLK>::XB + i) * BLK + __builtin_amdgcn_readfirstlane(threadIdx.x & ~(kWave - 1));
}

template <int Q, bool NORM, int BLK>
__device__ __forceinline__ void stage_issue(const GemvArgs& a, XStage<Q, NORM, BLK>& st, int batch, int NC) {
  using T = QTraits<Q>;
  const _Float16* x = reinterpret_cast<const _Float16*>(a.x);
  const _Float16* nw = reinterpret_cast<const _Float16*>(a.norm_w);
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int i = 0; i < XStage<Q, NORM, BLK>::XB; ++i) {
    const int c0 = stage_base<Q, NORM, BLK>(batch, i);
    if (c0 < NC) {
      const int c = min(c0 + lane, NC - 1);
#pragma unroll
      for (int p = 0; p < T::PLANES; ++p) {
        st.x[i][p] = load_u4(x + c * T::EPC + p * 8);
        if constexpr (NORM) st.w[i][p] = load_u4(nw + c * T::EPC + p * 8);
      }
    }
  }
}

template <int Q, bool NORM, int BLK>
__device__ __forceinline__ void stage_write(const XStage<Q, NORM, BLK>& st, int batch, int NC, u4_t* xs, float* sx) {
  using T = QTraits<Q>;
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int i = 0; i < XStage<Q, NORM, BLK>::XB; ++i) {
    const int c0 = stage_base<Q, NORM, BLK>(batch, i);
    if (c0 >= NC) continue;
    // lanes past the end write chunk NC-1 again with the identical value
    const int c = min(c0 + lane, NC - 1);
    float corr = 0.f;
    u4_t planes[T::PLANES];
#pragma unroll
    for (int p = 0; p < T::PLANES; ++p) {
      u4_t m = st.x[i][p];
      if constexpr (NORM) {
        // half(x * w) as one packed multiply per pair: the product of two
        // fp16 values is exact in fp32, so this rounds exactly like the
        // fp32 multiply and conversion
        const u4_t w = st.w[i][p];
        m.x = as_u32(as_h2(m.x) * as_h2(w.x));
        m.y = as_u32(as_h2(m.y) * as_h2(w.y));
        m.z = as_u32(as_h2(m.z) * as_h2(w.z));
        m.w = as_u32(as_h2(m.w) * as_h2(w.w));
      }
      corr += plane_order_packed<Q>(m, planes[p]);
    }
#pragma unroll
    for (int p = 0; p < T::PLANES; ++p) xs[p * NC + c] = planes[p];
    if constexpr (quantized<Q>()) sx[c] = corr;
  }
}

// Finishes the staging whose batch 0 was issued with stage_issue; returns
// the RMSNorm scale (1 without NORM).  `red` holds BLK/64 floats of LDS.
template <int Q, bool NORM, int BLK>
__device__ __forceinline__ float stage_finish(const GemvArgs& a, XStage<Q, NORM, BLK>& st, int NC, u4_t* xs, float* sx,
                                              float* red) {
  using T = QTraits<Q>;
  using XS = XStage<Q, NORM, BLK>;
  if constexpr (NORM) {
    // one batch holds all of x (host-checked)
    const int lane = threadIdx.x & (kWave - 1);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < XS::XB; ++i) {
      const int c0 = stage_base<Q, NORM, BLK>(0, i);
      if (c0 < NC && c0 + lane < NC) {
#pragma unroll
        for (int p = 0; p < T::PLANES; ++p) {
          const u4_t xv = st.x[i][p];
          ss = __builtin_amdgcn_fdot2(as_h2(xv.x), as_h2(xv.x), ss, false);
          ss = __builtin_amdgcn_fdot2(as_h2(xv.y), as_h2(xv.y), ss, false);
          ss = __builtin_amdgcn_fdot2(as_h2(xv.z), as_h2(xv.z), ss, false);
          ss = __builtin_amdgcn_fdot2(as_h2(xv.w), as_h2(xv.w), ss, false);
        }
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) red[threadIdx.x / kWave] = ss;
  }
  stage_write<Q, NORM, BLK>(st, 0, NC, xs, sx);
  if constexpr (!NORM) {   // with the norm fused, XB is sized so one batch holds all of x
    for (int b = 1; b * XS::XB * BLK < NC; ++b) {
      stage_issue<Q, NORM, BLK>(a, st, b, NC);
      stage_write<Q, NORM, BLK>(st, b, NC, xs, sx);
    }
  }
  __syncthreads();
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < BLK / kWave; ++w) ss += red[w];
    // eps travels as fp16 in the reference (kernels.cu:726, model.cu:96)
    return rsqrtf(ss / (float)a.K + (float)(_Float16)a.eps);
  }
  return 1.f;
}

// Rows handled by one wave unit.
template <int MODE, int R>
__host__ __device__ __forceinline__ int units_total(const GemvArgs& a) {
  if constexpr (MODE == GM_SWIGLU) return (a.N + R / 2 - 1) / (R / 2);
  else if constexpr (MODE == GM_QKV) return (a.n_heads + 2 * a.n_kv) * (a.head_dim / 2) / (R / 2);
  else return (a.N + R - 1) / R;
}

// Output rows of one SWIGLU unit: a block's contiguous unit range owns a
// contiguous slice of the output.
template <int MODE, int R>
__host__ __device__ constexpr int rows_per_unit() { return MODE == GM_SWIGLU ? R / 2 : R; }

// Pointer `i` of a 3-entry kernel-argument array.  Written as selects so the
// pointers stay in scalar registers; indexing the array with a run-time
// value makes the compiler re-load it from kernarg memory with a vector load
// and a full vmcnt(0) wait, which would serialise the prologue's loads.
template <typename T>
__device__ __forceinline__ T sel3(T const (&arr)[3], int i) {
  return i == 0 ? arr[0] : (i == 1 ? arr[1] : arr[2]);
}

struct RowRef {
  int mat;    // matrix index into a.W / a.S / a.bias / a.out
  int row;    // row within that matrix
  bool valid;
};

template <int MODE, int R>
__device__ __forceinline__ RowRef row_of(const GemvArgs& a, int unit, int r) {
  RowRef rr;
  if constexpr (MODE == GM_SWIGLU) {
    const int o = unit * (R / 2) + (r % (R / 2));
    rr.mat = r < R / 2 ? 0 : 1;
    rr.valid = o < a.N;
    rr.row = rr.valid ? o : a.N - 1;
  } else if constexpr (MODE == GM_QKV) {
    constexpr int PP = R / 2;
    const int half = a.head_dim / 2;
    const int per_head = half / PP;
    const int h = unit / per_head;
    const int p = (unit % per_head) * PP + (r % PP);
    const int within = p + (r < PP ? 0 : half);
    int mh;
    if (h < a.n_heads) { rr.mat = 0; mh = h; }
    else if (h < a.n_heads + a.n_kv) { rr.mat = 1; mh = h - a.n_heads; }
    else { rr.mat = 2; mh = h - a.n_heads - a.n_kv; }
    rr.row = mh * a.head_dim + within;
    rr.valid = true;
  } else {
    const int row = unit * R + r;
    rr.mat = 0;
    rr.valid = row < a.N;
    rr.row = rr.valid ? row : a.N - 1;
  }
  return rr;
}

// Per-wave register buffer of one k-step: kUnroll 16-byte chunks of R rows.
template <int R, int U>
struct StepBuf {
  u4_t w[U][R];
  _Float16 sc[U][R];   // converted at use, so the issue of the next step's loads never waits on them
};

// SWIGLU (several units per wave) runs the loop whose loads are issued on
// every path; the other modes keep the loop that skips the loads of steps
// past the wave's range (measured: QKV and the down projection, one unit
// per wave at 7B, were 0.5 and 0.9 us slower per launch with the former;
// the lm_head, 18 units per wave, unchanged).
template <int MODE>
__host__ __device__ constexpr bool gemv_buffer_loop() { return MODE == GM_SWIGLU; }

// The loads of one step, through buffer resources that are empty when the
// step is not real work (past the wave's range): the loop then issues the
// same loads on every path, so the compiler's waits name exactly the buffer
// being computed, and a step that is never used costs no memory round trip.
// The row offset is wave-uniform (soffset), the lane's chunk offset a vector.
template <int Q, int MODE, int R, int U, bool G128>
__device__ __forceinline__ void load_step(const GemvArgs& a, StepBuf<R, U>& b, int unit, int kb, int NC, int lane,
                                          bool real) {
  using T = QTraits<Q>;
  // 32-bit offsets (every matrix is below 2 GiB, host-checked): the
  // prologue's address arithmetic runs on the CU's one scalar unit for all
  // its waves at once, and 64-bit multiplies cost it several instructions each
  const uint32_t rbytes = (uint32_t)NC * 16u;
  const uint32_t sstride = G128 ? (uint32_t)(a.K / kGroup) : 1u;
  if constexpr (!gemv_buffer_loop<MODE>()) {
    // one-pass modes: plain global loads (a step past the range reads a
    // valid unit and is never issued by the loop)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const RowRef rr = row_of<MODE, R>(a, unit, r);
      const char* rp = reinterpret_cast<const char*>(sel3(a.W, rr.mat)) + (uint32_t)rr.row * rbytes;
      const _Float16* sp = nullptr;
      if constexpr (quantized<Q>()) sp = reinterpret_cast<const _Float16*>(sel3(a.S, rr.mat)) + (uint32_t)rr.row * sstride;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = min(kb * (kWave * U) + u * kWave + lane, NC - 1);
        b.w[u][r] = load_u4_stream(rp + (uint32_t)c * 16u);
        if constexpr (quantized<Q>()) b.sc[u][r] = sp[G128 ? (c * T::EPC) / kGroup : 0];
      }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const RowRef rr = row_of<MODE, R>(a, unit, r);
    const __amdgpu_buffer_rsrc_t rw = rsrc_or_null(sel3(a.W, rr.mat), real);
    const uint32_t roff = (uint32_t)rr.row * rbytes;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(kb * (kWave * U) + u * kWave + lane, NC - 1);
      b.w[u][r] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)c * 16u, roff, kCacheNT));
      if constexpr (quantized<Q>()) {
        const __amdgpu_buffer_rsrc_t rs = rsrc_or_null(sel3(a.S, rr.mat), real);
        const uint32_t si = G128 ? (uint32_t)(c * T::EPC) / kGroup : 0u;
        b.sc[u][r] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(rs, si * 2u, (uint32_t)rr.row * sstride * 2u, 0));
      }
    }
  }
}

template <int Q, int R, int U>
__device__ __forceinline__ void compute_step(const StepBuf<R, U>& b, float (&acc)[R], const u4_t* xs, const float* sx,
                                             int kb, int NC, int lane, const UnpackRegs& k) {
  using T = QTraits<Q>;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = kb * (kWave * U) + u * kWave + lane;
    if (c < NC) {
      u4_t xv[T::PLANES];
#pragma unroll
      for (int p = 0; p < T::PLANES; ++p) xv[p] = xs[p * NC + c];
      if constexpr (quantized<Q>()) {
        const float corr = sx[c];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = fmaf((float)b.sc[u][r], chunk_dot<Q>(b.w[u][r], xv, k) - corr, acc[r]);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += chunk_dot<Q>(b.w[u][r], xv, k);
      }
    }
  }
}

// Epilogue operands fetched together with a unit's first weights, so the
// epilogue does not start a dependent memory round trip: lane r < R holds
// the residual x[row] (RESID) or the bias and penalty stamp (STORE); in QKV
// mode lane i < R/2 holds the biases of its rotation pair.
struct EpiPre {
  uint32_t a = 0, b = 0;   // raw fp16 bits, zero-extended; converted where used
};
__device__ __forceinline__ float epi_f(uint32_t bits) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits); }
__device__ __forceinline__ uint32_t ld_u16(const void* p) { return *reinterpret_cast<const uint16_t*>(p); }

template <int MODE, int R>
__device__ __forceinline__ EpiPre epi_prefetch(const GemvArgs& a, int unit, int lane, bool /*real: SWIGLU loads nothing here*/) {
  // Every lane loads from a valid address (lanes past R re-read row R-1;
  // a missing bias reads x[0] and is ignored at use), so the loads are
  // unconditional and the compiler's load counters stay exact.
  EpiPre e;
  if constexpr (MODE == GM_STORE || MODE == GM_RESID) {
    const RowRef me = row_of<MODE, R>(a, unit, min(lane, R - 1));
    if constexpr (MODE == GM_RESID) {
      e.a = ld_u16(reinterpret_cast<const _Float16*>(a.resid ? a.resid : a.out[0]) + me.row);
    } else {
      e.a = ld_u16(a.bias[0] ? reinterpret_cast<const _Float16*>(a.bias[0]) + me.row
                             : reinterpret_cast<const _Float16*>(a.x));
      // the row's penalty stamp (a missing stamp array reads x[0..1], ignored at use)
      e.b = *(a.stamp ? a.stamp + me.row : reinterpret_cast<const uint32_t*>(a.x));
    }
  } else if constexpr (MODE == GM_QKV) {
    constexpr int PP = R / 2;
    const int i = min(lane, PP - 1);
    const RowRef r0 = row_of<MODE, R>(a, unit, i);
    const RowRef r1 = row_of<MODE, R>(a, unit, i + PP);
    const _Float16* b = reinterpret_cast<const _Float16*>(sel3(a.bias, r0.mat));
    const _Float16* x0 = reinterpret_cast<const _Float16*>(a.x);
    e.a = ld_u16(b ? b + r0.row : x0);
    e.b = ld_u16(b ? b + r1.row : x0);
  }
  return e;
}

// Epilogue of one output row (STORE / RESID modes); returns the stored
// value's argmax key.
template <int MODE, int R>
__device__ __forceinline__ unsigned long long store_row(const GemvArgs& a, float v, float pre, uint32_t stamp,
                                                        uint32_t epoch, int unit, int r) {
  const RowRef me = row_of<MODE, R>(a, unit, r);
  if (!me.valid) return 0ull;
  _Float16* out = reinterpret_cast<_Float16*>(a.out[0]);
  v += pre;   // residual (kernels.cu:621, :671: it stays fp16) or bias
  _Float16 h = (_Float16)v;
  if (MODE == GM_STORE && a.stamp && stamp == epoch) {
    // repetition penalty on the fp16 logit (kernels.cu:885-888)
    const float pen = (float)(_Float16)a.penalty;
    const float l = (float)h;
    h = (_Float16)(l < 0.f ? l * pen : l / pen);
  }
  out[me.row] = h;
  return argmax_key((float)h, me.row);   // the stored value, as the argmax reads it back
}

// QKV epilogue of one rotation pair (rows i and i + hd/2 of a head): bias,
// fp16, NeoX RoPE on q/k, k/v into the cache.  inv_freq[i] = theta^(-2i/hd)
// in double (a host-computed table staged in LDS); the angle pos * inv_freq
// is reduced modulo 2 pi in double and its sine and cosine taken in fp32.
template <int MODE, int R>
__device__ __forceinline__ void qkv_pair(const GemvArgs& a, float y0, float y1, const EpiPre& pre, int unit,
                                         int i_pair, const double* inv_freq, int pos) {
  constexpr int PP = R / 2;
  const RowRef r0 = row_of<MODE, R>(a, unit, i_pair);
  const RowRef r1 = row_of<MODE, R>(a, unit, i_pair + PP);
  const bool has_bias = sel3(a.bias, r0.mat) != nullptr;
  y0 = (float)(_Float16)(y0 + (has_bias ? epi_f(pre.a) : 0.f));   // q/k/v are fp16 before RoPE (kernels.cu:470)
  y1 = (float)(_Float16)(y1 + (has_bias ? epi_f(pre.b) : 0.f));
  const int hd = a.head_dim;
  if (r0.mat < 2) rope_rotate(y0, y1, pos, inv_freq[r0.row % hd]);   // q and k only
  const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1;
  _Float16* out = reinterpret_cast<_Float16*>(sel3(a.out, r0.mat));
  if (out) { out[r0.row] = h0; out[r1.row] = h1; }
  if (r0.mat > 0 && a.kcache) {
    const int kvh = r0.row / hd, d0 = r0.row % hd, d1 = r1.row % hd;
    _Float16* cache = reinterpret_cast<_Float16*>(r0.mat == 1 ? a.kcache : a.vcache);
    if (r0.mat == 1) {
      cache[kv_k_offset(kvh, pos, d0, a.max_seq, hd)] = h0;
      cache[kv_k_offset(kvh, pos, d1, a.max_seq, hd)] = h1;
    } else {
      cache[kv_v_offset(kvh, pos, d0, a.max_seq, hd)] = h0;
      cache[kv_v_offset(kvh, pos, d1, a.max_seq, hd)] = h1;
    }
  }
}

// Reduce the wave's R row sums, apply the RMSNorm scale, run the epilogue;
// lane r handles row r (static register indices only, so nothing goes
// through scratch).
template <int MODE, int R>
__device__ __forceinline__ void finish_unit(const GemvArgs& a, float (&acc)[R], int unit, int lane, float scale,
                                            const EpiPre& pre, const double* inv_freq, uint32_t step_word,
                                            unsigned long long& best, _Float16* stash, int row_base) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]) * scale;
  if constexpr (MODE == GM_STORE || MODE == GM_RESID) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (lane == r) {
        const unsigned long long k = store_row<MODE, R>(a, acc[r], (MODE == GM_RESID || a.bias[0]) ? epi_f(pre.a) : 0.f,
                                                        pre.b, step_word, unit, r);
        if constexpr (MODE == GM_STORE) best = k > best ? k : best;
      }
  } else if constexpr (MODE == GM_SWIGLU) {
#pragma unroll
    for (int r = 0; r < R / 2; ++r) {
      if (lane == r) {
        const RowRef me = row_of<MODE, R>(a, unit, r);
        if (me.valid) {
          const float g = acc[r], u = acc[r + R / 2];
          const float sig = 1.f / (1.f + expf(-g));    // kernels.cu:566
          stash[me.row - row_base] = (_Float16)((g * sig) * u);   // written out after the loop
        }
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < R / 2; ++r)
      if (lane == r) qkv_pair<MODE, R>(a, acc[r], acc[r + R / 2], pre, unit, r, inv_freq, (int)step_word);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
}

// Step cursor of one wave: which (unit, k-step) a step buffer holds and
// whether it is real work (a cursor past the block's range still names a
// valid unit, so its loads stay unconditional, but is never computed).
struct Cursor {
  int unit, kb;
  bool real;
};

}  // namespace cq
