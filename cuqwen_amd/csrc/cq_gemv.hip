// GEMV kernels and their launcher (see cq_gemv.h for the design).
#include "cq_gemv.h"
#include "cq_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

namespace cq {

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
  static constexpr int XB = NORM ? (kNormMaxK / QTraits<Q>::EPC + BLK - 1) / BLK : 1;
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
__device__ __forceinline__ int units_total(const GemvArgs& a) {
  if constexpr (MODE == GM_SWIGLU) return (a.N + R / 2 - 1) / (R / 2);
  else if constexpr (MODE == GM_QKV) return (a.n_heads + 2 * a.n_kv) * (a.head_dim / 2) / (R / 2);
  else return (a.N + R - 1) / R;
}

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

template <int Q, int MODE, int R, int U, bool G128>
__device__ __forceinline__ void load_step(const GemvArgs& a, StepBuf<R, U>& b, int unit, int kb, int NC, int lane) {
  using T = QTraits<Q>;
  const int64_t rbytes = (int64_t)NC * 16;
  const int sstride = G128 ? a.K / kGroup : 1;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const RowRef rr = row_of<MODE, R>(a, unit, r);
    const char* rp = reinterpret_cast<const char*>(sel3(a.W, rr.mat)) + (int64_t)rr.row * rbytes;
    const _Float16* sp = nullptr;
    if constexpr (quantized<Q>()) sp = reinterpret_cast<const _Float16*>(sel3(a.S, rr.mat)) + (int64_t)rr.row * sstride;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(kb * (kWave * U) + u * kWave + lane, NC - 1);
      b.w[u][r] = load_u4_stream(rp + (int64_t)c * 16);
      if constexpr (quantized<Q>()) b.sc[u][r] = sp[G128 ? (c * T::EPC) / kGroup : 0];
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
__device__ __forceinline__ EpiPre epi_prefetch(const GemvArgs& a, int unit, int lane) {
  // Every lane loads from a valid address (lanes past R re-read row R-1;
  // a missing bias reads x[0] and is ignored at use), so the loads are
  // unconditional and the compiler's load counters stay exact.
  EpiPre e;
  if constexpr (MODE == GM_STORE || MODE == GM_RESID) {
    const RowRef me = row_of<MODE, R>(a, unit, min(lane, R - 1));
    if constexpr (MODE == GM_RESID) {
      e.a = ld_u16(reinterpret_cast<const _Float16*>(a.out[0]) + me.row);
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
                                            unsigned long long& best) {
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
          reinterpret_cast<_Float16*>(a.out[0])[me.row] = (_Float16)((g * sig) * u);
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

// Persistent GEMV.  Block b owns the contiguous unit range
// [b*n/G, (b+1)*n/G); inside the block, wave w starts on units begin + w and
// begin + WPB + w and then claims further units from an LDS counter.  The
// claiming matters: a SIMD issues its oldest wave first, so with a static
// split the youngest waves of every SIMD finish far behind the oldest and
// the SIMD spends its last microseconds with few loads in flight; claimed
// units let early waves take over their share.  A step is U 16-byte chunks
// per lane of each of the unit's R rows.  Two step buffers rotate: while one
// step is reduced the next one's loads are in flight.  The first two steps
// (and their epilogue operands) are requested before the LDS staging so the
// input-vector prologue overlaps them.  The main loop issues loads only for
// real work, and unconditionally inside its body (clamped chunk indices),
// keeping the compiler's load counters exact.
template <int Q, int MODE, int R, int U, bool NORM, bool G128, int BLK>
__global__ __launch_bounds__(BLK) void gemv_kernel(const GemvArgs a) {
  using T = QTraits<Q>;
  extern __shared__ u4_t smem[];
  __shared__ float red[BLK / kWave];
  __shared__ double inv_freq[MODE == GM_QKV ? kMaxHeadDim / 2 : 1];
  __shared__ int next_unit;
  const int NC = a.K / T::EPC;
  u4_t* xs = smem;
  float* sx = reinterpret_cast<float*>(smem + T::PLANES * NC);
  const int lane = threadIdx.x & (kWave - 1);
  const int n_units = units_total<MODE, R>(a);
  constexpr int WPB = BLK / kWave;
  // wave index through readfirstlane: the compiler then knows every
  // per-unit quantity is wave-uniform and keeps the unit / k-step / row
  // address arithmetic in scalar registers (and the loop a scalar loop)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int u_begin = (int)(((int64_t)blockIdx.x * n_units) / gridDim.x);
  const int u_end = (int)(((int64_t)(blockIdx.x + 1) * n_units) / gridDim.x);
  const int u_last = max(u_end - 1, min(u_begin, n_units - 1));   // always a valid unit
  const int NB = (NC + kWave * U - 1) / (kWave * U);
  if (threadIdx.x == 0) next_unit = u_begin + 2 * WPB;   // published by the staging barrier

  auto make = [&](int unit, int kb) {
    Cursor c;
    c.real = unit < u_end;
    c.unit = c.real ? unit : u_last;
    c.kb = c.real ? kb : 0;
    return c;
  };
  // the step after c; `second` is the wave's second static unit (-1 once used)
  int second = u_begin + WPB + wave;
  auto advance = [&](const Cursor& c) {
    if (!c.real) return c;
    if (c.kb + 1 < NB) return make(c.unit, c.kb + 1);
    int u;
    if (second >= 0) {
      u = second;
      second = -1;
    } else {
      int v = 0;
      if (lane == 0) v = atomicAdd(&next_unit, 1);
      u = __builtin_amdgcn_readfirstlane(v);
    }
    return make(u, 0);
  };

  // The x loads go out at raised wave priority so that every resident
  // wave's staging loads are issued before any wave's weight prefetch:
  // the CU's memory pipeline serves loads in issue order, and x behind the
  // weights would hold the staging barrier for a full weight round trip.
  __builtin_amdgcn_s_setprio(3);
  XStage<Q, NORM, BLK> st;
  stage_issue<Q, NORM, BLK>(a, st, 0, NC);
  // the RoPE table rides with the x loads (every thread, clamped index):
  // waiting for a load issued after the weight prefetch would wait for the
  // whole prefetch
  double rope_f = 0.0;
  if constexpr (MODE == GM_QKV) rope_f = a.rope_inv_freq[min((int)threadIdx.x, a.head_dim / 2 - 1)];
  // the step's control word the epilogue needs (QKV: position; STORE: the
  // penalty epoch), also read up front rather than in the epilogue
  uint32_t step_word = 0;
  if constexpr (MODE == GM_QKV) step_word = (uint32_t)*a.d_pos;
  if constexpr (MODE == GM_STORE) step_word = a.stamp ? *a.d_epoch : 0u;
  __builtin_amdgcn_s_setprio(0);
  StepBuf<R, U> A, B;
  Cursor ca = make(u_begin + wave, 0);
  Cursor cb = advance(ca);   // never claims: the first unit's next step or the second static unit
  // the first two steps are requested unconditionally (a cursor past the
  // range reads a valid unit that is never used)
  load_step<Q, MODE, R, U, G128>(a, A, ca.unit, ca.kb, NC, lane);
  EpiPre pa = epi_prefetch<MODE, R>(a, ca.unit, lane);
  load_step<Q, MODE, R, U, G128>(a, B, cb.unit, cb.kb, NC, lane);
  EpiPre pb = epi_prefetch<MODE, R>(a, cb.unit, lane);
  if constexpr (MODE == GM_QKV) inv_freq[min((int)threadIdx.x, a.head_dim / 2 - 1)] = rope_f;   // duplicates write equal values
  const float scale = stage_finish<Q, NORM, BLK>(a, st, NC, xs, sx, red);

  const UnpackRegs uk = unpack_regs();
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  unsigned long long best = 0ull;   // STORE: argmax key of the rows this lane stored
  auto run_a = [&]() {
    compute_step<Q, R, U>(A, acc, xs, sx, ca.kb, NC, lane, uk);
    if (ca.kb == NB - 1) finish_unit<MODE, R>(a, acc, ca.unit, lane, scale, pa, inv_freq, step_word, best);
  };
  auto run_b = [&]() {
    compute_step<Q, R, U>(B, acc, xs, sx, cb.kb, NC, lane, uk);
    if (cb.kb == NB - 1) finish_unit<MODE, R>(a, acc, cb.unit, lane, scale, pb, inv_freq, step_word, best);
  };
  // Steady state: A and B both hold real steps and each round refills both,
  // so every load in the loop is unconditional and the compiler's load
  // counters stay exact.  When the next step is past the wave's range the
  // wave leaves the loop before issuing its loads (a load whose data is
  // never used would still hold the wave until it returned) and finishes the
  // buffer it still holds.
  if (ca.real) {
    if (!cb.real) {
      run_a();
    } else {
      while (true) {
        run_a();
        const Cursor na = advance(cb);
        if (!na.real) {
          run_b();
          break;
        }
        ca = na;
        load_step<Q, MODE, R, U, G128>(a, A, ca.unit, ca.kb, NC, lane);
        pa = epi_prefetch<MODE, R>(a, ca.unit, lane);
        run_b();
        const Cursor nb = advance(ca);
        if (!nb.real) {
          run_a();
          break;
        }
        cb = nb;
        load_step<Q, MODE, R, U, G128>(a, B, cb.unit, cb.kb, NC, lane);
        pb = epi_prefetch<MODE, R>(a, cb.unit, lane);
      }
    }
  }
  if constexpr (MODE == GM_STORE) {
    // every launched wave writes its slot (0 when it stored nothing)
    if (a.argmax_out) {
      best = wave_max_u64(best);
      if (lane == 0) a.argmax_out[blockIdx.x * WPB + wave] = best;
    }
  }
}

// ------------------------------------------------------------------ host
void rope_inv_freq_host(float theta, int head_dim, double* out) {
  for (int i = 0; i < head_dim / 2; ++i) out[i] = 1.0 / std::pow((double)theta, (2.0 * i) / (double)head_dim);
}

int rope_table(float theta, int head_dim, const double** out) {
  static std::mutex mu;
  static std::map<std::tuple<int, uint32_t, int>, double*> tables;
  if (head_dim <= 0 || head_dim > kMaxHeadDim || head_dim % 2) return fail(CQ_EINVAL, "rope: bad head_dim");
  int dev = 0;
  CQ_HIP(hipGetDevice(&dev));
  uint32_t tbits;
  std::memcpy(&tbits, &theta, 4);
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dev, tbits, head_dim);
  auto it = tables.find(key);
  if (it != tables.end()) {
    *out = it->second;
    return CQ_OK;
  }
  double host[kMaxHeadDim / 2];
  rope_inv_freq_host(theta, head_dim, host);
  double* d = nullptr;
  CQ_HIP(hipMalloc(&d, sizeof host));
  const hipError_t e = hipMemcpy(d, host, sizeof(double) * (head_dim / 2), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return fail(CQ_EHIP, std::string("rope: table upload failed: ") + hipGetErrorString(e));
  }
  tables.emplace(key, d);
  *out = d;
  return CQ_OK;
}

int gemv_check(const GemvArgs& a) {
  if (a.quant < 0 || a.quant > 2) return fail(CQ_EINVAL, "gemv: bad quant type");
  if (a.K <= 0 || a.N <= 0) return fail(CQ_EINVAL, "gemv: empty shape");
  if (a.quant != CQ_QUANT_FP16 && a.K % kGroup) return fail(CQ_EINVAL, "gemv: cols must be a multiple of 128 for quantized weights");
  if (a.K % 8) return fail(CQ_EINVAL, "gemv: cols must be a multiple of 8");
  if (a.group != kGroup && a.group != 0) return fail(CQ_EINVAL, "gemv: group size must be 128 or 0 (per row)");
  if (!a.x || !a.W[0]) return fail(CQ_EINVAL, "gemv: null input");
  if (a.quant != CQ_QUANT_FP16 && !a.S[0]) return fail(CQ_EINVAL, "gemv: quantized weights need scales");
  if (a.mode == GM_SWIGLU && (!a.W[1] || (a.quant != CQ_QUANT_FP16 && !a.S[1])))
    return fail(CQ_EINVAL, "gemv: swiglu needs gate and up");
  if (a.mode == GM_QKV) {
    if (a.head_dim % 4 || a.head_dim > kMaxHeadDim || a.n_heads <= 0 || a.n_kv <= 0 || a.n_heads % a.n_kv)
      return fail(CQ_EINVAL, "gemv: bad head configuration");
    if (!a.W[1] || !a.W[2] || !a.d_pos || !a.rope_inv_freq)
      return fail(CQ_EINVAL, "gemv: qkv needs q, k, v weights, d_pos and the RoPE table");
    if (a.quant != CQ_QUANT_FP16 && (!a.S[1] || !a.S[2])) return fail(CQ_EINVAL, "gemv: qkv needs q, k, v scales");
    if (a.kcache && a.max_seq % 32) return fail(CQ_EINVAL, "gemv: max_seq must be a multiple of 32");
  } else if (!a.out[0]) {
    return fail(CQ_EINVAL, "gemv: null output");
  }
  const int planes = a.quant == CQ_QUANT_INT4 ? 4 : a.quant == CQ_QUANT_INT8 ? 2 : 1;
  const int epc = a.quant == CQ_QUANT_INT4 ? 32 : a.quant == CQ_QUANT_INT8 ? 16 : 8;
  const size_t lds = (size_t)planes * (a.K / epc) * 16 + (a.quant ? (size_t)(a.K / epc) * 4 : 0);
  if (lds > 60 * 1024) return fail(CQ_EINVAL, "gemv: input vector too long for LDS staging");
  if (a.norm_w && a.K > kNormMaxK) return fail(CQ_EINVAL, "gemv: fused RMSNorm supports K <= 16384");
  if (a.argmax_out && a.mode != GM_STORE) return fail(CQ_EINVAL, "gemv: argmax keys need the store mode");
  return CQ_OK;
}

// Tuning of one launch (measured on MI355X at the Qwen2.5-7B INT4 shapes):
// rows per wave, 16-byte chunks per lane per step, threads per block, and
// resident blocks per CU of the persistent grid.
// Fat 1024-thread blocks stage x once per CU for the long GEMVs; the short
// QKV projection prefers more, smaller blocks.
template <int MODE> struct GemvTune;
template <> struct GemvTune<GM_STORE> { static constexpr int R = 2, U = 2, BLK = 1024, PER_CU = 1; };
template <> struct GemvTune<GM_RESID> { static constexpr int R = 1, U = 2, BLK = 1024, PER_CU = 1; };
template <> struct GemvTune<GM_SWIGLU> { static constexpr int R = 2, U = 1, BLK = 1024, PER_CU = 1; };
template <> struct GemvTune<GM_QKV> { static constexpr int R = 2, U = 1, BLK = 256, PER_CU = 4; };

template <int Q, int MODE, int R, int U, bool NORM, bool G128, int BLK = 256>
int launch_variant(const GemvArgs& a, hipStream_t stream, int max_blocks) {
  constexpr int kWavesPerBlock = BLK / kWave;
  using T = QTraits<Q>;
  const int NC = a.K / T::EPC;
  const size_t lds = (size_t)T::PLANES * NC * 16 + (Q != CQ_QUANT_FP16 ? (size_t)NC * 4 : 0);
  int units;
  if (MODE == GM_SWIGLU) units = (a.N + R / 2 - 1) / (R / 2);
  else if (MODE == GM_QKV) units = (a.n_heads + 2 * a.n_kv) * (a.head_dim / 2) / (R / 2);
  else units = (a.N + R - 1) / R;
  // persistent grid: up to max_blocks blocks, each owning a contiguous range
  // of at least one unit per wave
  const int blocks = std::max(1, std::min(max_blocks, (units + kWavesPerBlock - 1) / kWavesPerBlock));
  if (a.argmax_out && blocks * kWavesPerBlock > kArgmaxPartials) return fail(CQ_EINVAL, "gemv: too many waves for the argmax slots");
  hipLaunchKernelGGL((gemv_kernel<Q, MODE, R, U, NORM, G128, BLK>), dim3(blocks), dim3(BLK), lds, stream, a);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

template <int Q, int MODE, bool NORM, bool G128>
static int launch_t(const GemvArgs& a, hipStream_t stream) {
  using TN = GemvTune<MODE>;
  return launch_variant<Q, MODE, TN::R, TN::U, NORM, G128, TN::BLK>(a, stream, TN::PER_CU * kNumCUs);
}

template <int Q, int MODE>
static int launch_q(const GemvArgs& a, hipStream_t stream) {
  const bool norm = a.norm_w != nullptr;
  if constexpr (MODE == GM_STORE) {
    // Short matrices (e.g. the 896-row down-projection shape of BASELINE
    // config 1) need more, smaller blocks than the 150K-row lm_head.
    if (a.N < 16384 && !norm) {
      if (a.group == 0) return launch_variant<Q, MODE, 2, 2, false, false, 256>(a, stream, 4 * kNumCUs);
      return launch_variant<Q, MODE, 2, 2, false, true, 256>(a, stream, 4 * kNumCUs);
    }
    if (a.group == 0) return norm ? launch_t<Q, MODE, true, false>(a, stream) : launch_t<Q, MODE, false, false>(a, stream);
    return norm ? launch_t<Q, MODE, true, true>(a, stream) : launch_t<Q, MODE, false, true>(a, stream);
  } else if constexpr (MODE == GM_RESID) {
    if (norm) return fail(CQ_EINVAL, "gemv: residual mode takes no norm");
    // short rows (at most two 64-chunk steps, e.g. the 7B o_proj) stream
    // faster one chunk per lane per step; long rows (down) two
    if (a.K / QTraits<Q>::EPC <= 2 * kWave) {
      using TN = GemvTune<MODE>;
      return launch_variant<Q, MODE, TN::R, 1, false, true, TN::BLK>(a, stream, TN::PER_CU * kNumCUs);
    }
    return launch_t<Q, MODE, false, true>(a, stream);
  } else {
    return norm ? launch_t<Q, MODE, true, true>(a, stream) : launch_t<Q, MODE, false, true>(a, stream);
  }
}

template <int Q>
static int launch_mode(const GemvArgs& a, hipStream_t stream) {
  switch (a.mode) {
    case GM_STORE: return launch_q<Q, GM_STORE>(a, stream);
    case GM_RESID: return launch_q<Q, GM_RESID>(a, stream);
    case GM_SWIGLU: return launch_q<Q, GM_SWIGLU>(a, stream);
    case GM_QKV: return launch_q<Q, GM_QKV>(a, stream);
  }
  return fail(CQ_EINVAL, "gemv: bad mode");
}

int launch_gemv(const GemvArgs& a, hipStream_t stream) {
  CQ_TRY(gemv_check(a));
  switch (a.quant) {
    case CQ_QUANT_FP16: return launch_mode<CQ_QUANT_FP16>(a, stream);
    case CQ_QUANT_INT8: return launch_mode<CQ_QUANT_INT8>(a, stream);
    default: return launch_mode<CQ_QUANT_INT4>(a, stream);
  }
}

// ------------------------------------------------------------- dequantize
// out[r][k] = q * scale through the same unpack helpers as the GEMV (test
// hook for the bit-exact unpack check).  One thread per 16-byte chunk.
template <int Q>
__global__ void dequant_kernel(const char* W, const _Float16* S, float* out, int rows, int cols, int group) {
  using T = QTraits<Q>;
  const int nc = cols / T::EPC;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)rows * nc) return;
  const int r = (int)(id / nc), c = (int)(id % nc);
  const u4_t w = load_u4(W + ((int64_t)r * nc + c) * 16);
  const float s = group ? (float)S[(int64_t)r * (cols / group) + (c * T::EPC) / group] : (float)S[r];
  float* o = out + (int64_t)r * cols + (int64_t)c * T::EPC;
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  const UnpackRegs k = unpack_regs();
  if constexpr (Q == CQ_QUANT_INT4) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t f = words[p] ^ kInt4Flip, f8 = f >> 8;
      const h2_t a0 = as_h2(and_or(f, k.m_lo, 0x64006400u)), a1 = as_h2(and_or(f, k.m_hi, 0x64006400u));
      const h2_t a2 = as_h2(and_or(f8, k.m_lo, 0x64006400u)), a3 = as_h2(and_or(f8, k.m_hi, 0x64006400u));
      // (1024 + n) - 1032 = q ; (1024 + 16 n) / 16 - 72 = q
      o[8 * p + 0] = ((float)a0.x - kInt4BiasLo) * s;
      o[8 * p + 4] = ((float)a0.y - kInt4BiasLo) * s;
      o[8 * p + 1] = ((float)a1.x * 0.0625f - kInt4BiasHi) * s;
      o[8 * p + 5] = ((float)a1.y * 0.0625f - kInt4BiasHi) * s;
      o[8 * p + 2] = ((float)a2.x - kInt4BiasLo) * s;
      o[8 * p + 6] = ((float)a2.y - kInt4BiasLo) * s;
      o[8 * p + 3] = ((float)a3.x * 0.0625f - kInt4BiasHi) * s;
      o[8 * p + 7] = ((float)a3.y * 0.0625f - kInt4BiasHi) * s;
    }
  } else {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t f = words[p] ^ kInt8Flip;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const h2_t h = as_h2(int8_pair(f, k.magic, i));
        o[4 * p + 2 * i] = ((float)h.x - kInt8Bias) * s;
        o[4 * p + 2 * i + 1] = ((float)h.y - kInt8Bias) * s;
      }
    }
  }
}

int launch_dequant(int quant, int group, const void* W, const __half* S, float* out, int rows, int cols,
                   hipStream_t stream) {
  if (quant != CQ_QUANT_INT8 && quant != CQ_QUANT_INT4) return fail(CQ_EINVAL, "dequant: quantized types only");
  if (cols % kGroup || rows <= 0 || (group != 0 && group != kGroup)) return fail(CQ_EINVAL, "dequant: bad shape");
  const int epc = quant == CQ_QUANT_INT4 ? 32 : 16;
  const int64_t n = (int64_t)rows * (cols / epc);
  const int blocks = (int)((n + 255) / 256);
  if (quant == CQ_QUANT_INT4)
    hipLaunchKernelGGL(dequant_kernel<CQ_QUANT_INT4>, dim3(blocks), dim3(256), 0, stream, (const char*)W,
                       (const _Float16*)S, out, rows, cols, group);
  else
    hipLaunchKernelGGL(dequant_kernel<CQ_QUANT_INT8>, dim3(blocks), dim3(256), 0, stream, (const char*)W,
                       (const _Float16*)S, out, rows, cols, group);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

}  // namespace cq
