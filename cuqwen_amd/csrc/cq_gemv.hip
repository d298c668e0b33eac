// GEMV kernels and their launcher (see cq_gemv.h for the design).
#include "cq_gemv.h"
#include "cq_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>

namespace cq {

// Value of a 64-bit fixed-point sum (2^-32 units, |value| < 2^30 by the
// producer's clamp) from its low and high words: the signed high word
// converts in one instruction (exactly below 2^24), the low word adds its
// fraction in one fma.  A full int64 conversion has no instruction and would
// cost the staging waves tens of instructions per element.
__device__ __forceinline__ float fix_to_float(uint32_t lo, uint32_t hi) {
  return fmaf((float)lo, 2.3283064365386963e-10f, (float)(int32_t)hi);
}

// Every kernel-argument word a mode reads, fetched in one batch of scalar
// loads at entry (CQ_PIN): the GEMV prologue otherwise waited for three or
// four dependent kernel-argument round trips between its address
// computations before the weight prefetch was out.
template <int Q, int MODE, bool NORM, bool ADD>
__device__ __forceinline__ void pin_args(const GemvArgs& a) {
  CQ_PIN(gridDim.x);   // an implicit kernel argument
  CQ_PIN(a.x); CQ_PIN(a.K); CQ_PIN(a.N); CQ_PIN(a.W[0]); CQ_PIN(a.out[0]);
  if constexpr (Q != CQ_QUANT_FP16) CQ_PIN(a.S[0]);
  if constexpr (NORM) { CQ_PIN(a.norm_w); CQ_PIN(a.eps); }
  if constexpr (MODE == GM_SWIGLU || MODE == GM_QKV) {
    CQ_PIN(a.W[1]);
    if constexpr (Q != CQ_QUANT_FP16) CQ_PIN(a.S[1]);
  }
  if constexpr (MODE == GM_QKV) {
    CQ_PIN(a.W[2]); CQ_PIN(a.bias[0]); CQ_PIN(a.bias[1]); CQ_PIN(a.bias[2]);
    CQ_PIN(a.out[1]); CQ_PIN(a.out[2]);
    if constexpr (Q != CQ_QUANT_FP16) CQ_PIN(a.S[2]);
    CQ_PIN(a.n_heads); CQ_PIN(a.n_kv); CQ_PIN(a.head_dim); CQ_PIN(a.d_pos); CQ_PIN(a.rope_inv_freq);
    CQ_PIN(a.rope_theta);
    CQ_PIN(a.kcache); CQ_PIN(a.vcache); CQ_PIN(a.max_seq);
  }
  if constexpr (MODE == GM_STORE) {
    CQ_PIN(a.bias[0]); CQ_PIN(a.stamp); CQ_PIN(a.d_epoch); CQ_PIN(a.argmax_out); CQ_PIN(a.penalty);
  }
  if constexpr (MODE == GM_RESID) { CQ_PIN(a.resid); CQ_PIN(a.zero); CQ_PIN(a.zero_n); }
  if constexpr (ADD) { CQ_PIN(a.x_acc); CQ_PIN(a.x_out); }
}

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
//
// ADD (SWIGLU with the norm fused): x is first replaced by half(x + x_acc *
// 2^-32), the residual plus the O-projection's fixed-point sum
// (cq_omerge.hip; rounded as kernels.cu:671 rounds the residual add); the
// sums ride in the staging registers next to x, and h is written back to
// x_out, a chunk per block.
template <int Q, int MODE, int R, int U, bool NORM, bool G128, int BLK, bool ADD = false>
__global__ __launch_bounds__(BLK) void gemv_kernel(const GemvArgs a) {
  static_assert(!ADD || (NORM && MODE == GM_SWIGLU), "ADD is the norm-fused SWIGLU prologue");
  using T = QTraits<Q>;
  pin_args<Q, MODE, NORM, ADD>(a);
  extern __shared__ u4_t smem[];
  __shared__ float red[BLK / kWave];
  __shared__ double inv_freq[MODE == GM_QKV ? kMaxHeadDim / 2 : 1];
  __shared__ int next_unit;
  const int NC = a.K / T::EPC;
  u4_t* xs = smem;
  float* sx = reinterpret_cast<float*>(smem + T::PLANES * NC);
  // SWIGLU: the block's output rows are collected in LDS and written after
  // the loop.  A global store inside the loop, issued only
  // when a unit finishes, is counted by vmcnt like the loads, and the
  // compiler's waits after such a branch then also wait for the next step's
  // weight loads, leaving the wave with nothing in flight while it computes.
  _Float16* stash = reinterpret_cast<_Float16*>(sx + (Q != CQ_QUANT_FP16 ? NC : 0));
  const int lane = threadIdx.x & (kWave - 1);
  const int n_units = units_total<MODE, R>(a);
  constexpr int WPB = BLK / kWave;
  // wave index through readfirstlane: the compiler then knows every
  // per-unit quantity is wave-uniform and keeps the unit / k-step / row
  // address arithmetic in scalar registers (and the loop a scalar loop)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  // 32-bit: n_units * gridDim.x < 2^31 (host-checked)
  const int u_begin = (int)((blockIdx.x * (uint32_t)n_units) / gridDim.x);
  const int u_end = (int)(((blockIdx.x + 1) * (uint32_t)n_units) / gridDim.x);
  const int u_last = max(u_end - 1, min(u_begin, n_units - 1));   // always a valid unit
  const int NB = (NC + kWave * U - 1) / (kWave * U);
  constexpr int RPU = rows_per_unit<MODE, R>();
  const int row_base = u_begin * RPU;
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
  // ADD: the fixed-point sums of the same elements (8 bytes each, two per
  // 16-byte load), next to x in the staging registers
  constexpr int XB = XStage<Q, NORM, BLK>::XB;
  u4_t xacc[ADD ? XB : 1][ADD ? T::PLANES : 1][4];
  if constexpr (ADD) {
#pragma unroll
    for (int i = 0; i < XB; ++i) {
      const int c0 = stage_base<Q, NORM, BLK>(0, i);
      if (c0 < NC) {
        const int c = min(c0 + lane, NC - 1);
#pragma unroll
        for (int p = 0; p < T::PLANES; ++p)
#pragma unroll
          for (int q = 0; q < 4; ++q) xacc[i][p][q] = load_u4(a.x_acc + c * T::EPC + p * 8 + 2 * q);
      }
    }
  }
  // the RoPE table rides with the x loads (every thread, clamped index):
  // waiting for a load issued after the weight prefetch would wait for the
  // whole prefetch
  double rope_f = 0.0;
  if constexpr (MODE == GM_QKV) {
    const int i = min((int)threadIdx.x, a.head_dim / 2 - 1);
    rope_f = a.rope_inv_freq ? a.rope_inv_freq[i] : rope_inv_freq_dev(a.rope_theta, i, a.head_dim);
  }
  // the step's control word the epilogue needs (QKV: position; STORE: the
  // penalty epoch), also read up front rather than in the epilogue
  uint32_t step_word = 0;
  if constexpr (MODE == GM_QKV) step_word = load_ctl_u32(a.d_pos);
  if constexpr (MODE == GM_STORE) step_word = a.stamp ? load_ctl_u32(a.d_epoch) : 0u;
  __builtin_amdgcn_s_setprio(0);
  StepBuf<R, U> A, B;
  Cursor ca = make(u_begin + wave, 0);
  Cursor cb = advance(ca);   // never claims: the first unit's next step or the second static unit
  // the first two steps are requested unconditionally (a cursor past the
  // range names a valid unit and loads zeros without a memory access)
  load_step<Q, MODE, R, U, G128>(a, A, ca.unit, ca.kb, NC, lane, ca.real);
  EpiPre pa = epi_prefetch<MODE, R>(a, ca.unit, lane, ca.real);
  load_step<Q, MODE, R, U, G128>(a, B, cb.unit, cb.kb, NC, lane, cb.real);
  EpiPre pb = epi_prefetch<MODE, R>(a, cb.unit, lane, cb.real);
  if constexpr (MODE == GM_QKV) inv_freq[min((int)threadIdx.x, a.head_dim / 2 - 1)] = rope_f;   // duplicates write equal values
  if constexpr (ADD) {
    // h = half(x + sum): the O-projection sum (fp32) plus the fp16
    // residual, rounded once
#pragma unroll
    for (int i = 0; i < XB; ++i) {
      if (stage_base<Q, NORM, BLK>(0, i) < NC) {
#pragma unroll
        for (int p = 0; p < T::PLANES; ++p) {
          uint32_t w[4] = {st.x[i][p].x, st.x[i][p].y, st.x[i][p].z, st.x[i][p].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const u4_t s4 = xacc[i][p][q];
            const float o0 = fix_to_float(s4.x, s4.y);
            const float o1 = fix_to_float(s4.z, s4.w);
            const h2_t xv = as_h2(w[q]);
            h2_t h;
            h.x = (_Float16)(o0 + (float)xv.x);
            h.y = (_Float16)(o1 + (float)xv.y);
            w[q] = as_u32(h);
          }
          st.x[i][p] = u4_t{w[0], w[1], w[2], w[3]};
        }
      }
    }
  }
  const float scale = stage_finish<Q, NORM, BLK>(a, st, NC, xs, sx, red);
  if constexpr (ADD) {
    // chunk c of h is written by block c % gridDim.x (after the staging
    // barrier: a store pending at a barrier could make it wait for the
    // weight loads too)
#pragma unroll
    for (int i = 0; i < XB; ++i) {
      const int c = stage_base<Q, NORM, BLK>(0, i) + lane;
      if (c < NC && c % (int)gridDim.x == (int)blockIdx.x) {
#pragma unroll
        for (int p = 0; p < T::PLANES; ++p) *reinterpret_cast<u4_t*>(a.x_out + c * T::EPC + p * 8) = st.x[i][p];
      }
    }
  }

  const UnpackRegs uk = unpack_regs();
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  unsigned long long best = 0ull;   // STORE: argmax key of the rows this lane stored
  auto run_a = [&]() {
    compute_step<Q, R, U>(A, acc, xs, sx, ca.kb, NC, lane, uk);
    if (ca.kb == NB - 1) finish_unit<MODE, R>(a, acc, ca.unit, lane, scale, pa, inv_freq, step_word, best, stash, row_base);
  };
  auto run_b = [&]() {
    compute_step<Q, R, U>(B, acc, xs, sx, cb.kb, NC, lane, uk);
    if (cb.kb == NB - 1) finish_unit<MODE, R>(a, acc, cb.unit, lane, scale, pb, inv_freq, step_word, best, stash, row_base);
  };
  if constexpr (gemv_buffer_loop<MODE>()) {
    // A and B alternate; every half-round computes one buffer and refills it
    // with the step after the other one, unconditionally (a step past the
    // wave's range loads zeros without a memory access), so each compute
    // waits for its own buffer only while the other one's loads stay in flight.
    while (ca.real) {
      run_a();
      ca = advance(cb);
      load_step<Q, MODE, R, U, G128>(a, A, ca.unit, ca.kb, NC, lane, ca.real);
      pa = epi_prefetch<MODE, R>(a, ca.unit, lane, ca.real);
      if (!cb.real) break;
      run_b();
      cb = advance(ca);
      load_step<Q, MODE, R, U, G128>(a, B, cb.unit, cb.kb, NC, lane, cb.real);
      pb = epi_prefetch<MODE, R>(a, cb.unit, lane, cb.real);
    }
  } else {
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
          load_step<Q, MODE, R, U, G128>(a, A, ca.unit, ca.kb, NC, lane, true);
          pa = epi_prefetch<MODE, R>(a, ca.unit, lane, true);
          run_b();
          const Cursor nb = advance(ca);
          if (!nb.real) {
            run_a();
            break;
          }
          cb = nb;
          load_step<Q, MODE, R, U, G128>(a, B, cb.unit, cb.kb, NC, lane, true);
          pb = epi_prefetch<MODE, R>(a, cb.unit, lane, true);
        }
      }
    }
  }
  if constexpr (MODE == GM_SWIGLU) {
    __syncthreads();
    _Float16* out = reinterpret_cast<_Float16*>(a.out[0]);
    const int row_end = min(u_end * RPU, a.N);
    for (int i = row_base + (int)threadIdx.x; i < row_end; i += BLK) out[i] = stash[i - row_base];
  }
  if constexpr (MODE == GM_RESID) {
    if (a.zero)
      for (int i = blockIdx.x * BLK + threadIdx.x; i < a.zero_n; i += gridDim.x * BLK) a.zero[i] = 0;
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
    if (!a.W[1] || !a.W[2] || !a.d_pos) return fail(CQ_EINVAL, "gemv: qkv needs q, k, v weights and d_pos");
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
  // the kernel's address and unit arithmetic is 32-bit
  if ((int64_t)a.N * a.K * (a.quant == CQ_QUANT_FP16 ? 2 : 1) >= ((int64_t)1 << 31) || (int64_t)a.N * 2 * kNumCUs * 16 >= ((int64_t)1 << 31))
    return fail(CQ_EINVAL, "gemv: matrix too large (2 GiB per weight matrix)");
  if (a.x_acc && (a.mode != GM_SWIGLU || !a.norm_w || !a.x_out))
    return fail(CQ_EINVAL, "gemv: the accumulator prologue needs swiglu, a fused norm and x_out");
  if ((a.resid || a.zero) && a.mode != GM_RESID) return fail(CQ_EINVAL, "gemv: resid / zero are residual-mode options");
  if (a.zero_n < 0 || (a.zero_n > 0 && !a.zero)) return fail(CQ_EINVAL, "gemv: bad zero range");
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

template <int Q, int MODE, int R, int U, bool NORM, bool G128, int BLK = 256, bool ADD = false>
int launch_variant(const GemvArgs& a, hipStream_t stream, int max_blocks) {
  constexpr int kWavesPerBlock = BLK / kWave;
  using T = QTraits<Q>;
  const int NC = a.K / T::EPC;
  const int units = units_total<MODE, R>(a);
  // persistent grid: up to max_blocks blocks, each owning a contiguous range
  // of at least one unit per wave
  const int blocks = std::max(1, std::min(max_blocks, (units + kWavesPerBlock - 1) / kWavesPerBlock));
  // staged x (+ scales) and the output stash of the block's rows
  const size_t stash = MODE != GM_SWIGLU ? 0 : (size_t)((units + blocks - 1) / blocks) * rows_per_unit<MODE, R>() * 2;
  const size_t lds = (size_t)T::PLANES * NC * 16 + (Q != CQ_QUANT_FP16 ? (size_t)NC * 4 : 0) + stash;
  if (lds > 64 * 1024) return fail(CQ_EINVAL, "gemv: input vector and output slice too long for LDS");
  if (a.argmax_out && blocks * kWavesPerBlock > kArgmaxPartials) return fail(CQ_EINVAL, "gemv: too many waves for the argmax slots");
  hipLaunchKernelGGL((gemv_kernel<Q, MODE, R, U, NORM, G128, BLK, ADD>), dim3(blocks), dim3(BLK), lds, stream, a);
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
    // config 1) need more, smaller blocks than the 150K-row lm_head, and one
    // row per wave in few, wide steps (measured at K=4864 N=896 W8: R=1 U=3
    // 4.13 us per launch, R=2 U=2 4.92, R=1 U=5 4.21).
    if (a.N < 16384 && !norm) {
      if (a.group == 0) return launch_variant<Q, MODE, 1, 3, false, false, 256>(a, stream, 4 * kNumCUs);
      return launch_variant<Q, MODE, 1, 3, false, true, 256>(a, stream, 4 * kNumCUs);
    }
    if (a.group == 0) return norm ? launch_t<Q, MODE, true, false>(a, stream) : launch_t<Q, MODE, false, false>(a, stream);
    return norm ? launch_t<Q, MODE, true, true>(a, stream) : launch_t<Q, MODE, false, true>(a, stream);
  } else if constexpr (MODE == GM_RESID) {
    if (norm) return fail(CQ_EINVAL, "gemv: residual mode takes no norm");
    // Few rows (the 0.5B / 1.5B projections, N < 2048): 1024-thread blocks
    // would leave most CUs idle (896 rows = 56 blocks); 512-thread blocks,
    // two per CU (measured decode step 0.5B INT8 666 -> 640 us, 1.5B INT4
    // 965 -> 931 us; the 3584-row 7B shapes are faster with the fat blocks).
    if (a.N < 2048) {
      if (a.K / QTraits<Q>::EPC <= 2 * kWave) return launch_variant<Q, MODE, 1, 1, false, true, 512>(a, stream, 2 * kNumCUs);
      return launch_variant<Q, MODE, 1, 2, false, true, 512>(a, stream, 2 * kNumCUs);
    }
    // short rows (at most two 64-chunk steps, e.g. the 7B o_proj) stream
    // faster one chunk per lane per step; long rows (down) two
    if (a.K / QTraits<Q>::EPC <= 2 * kWave) {
      using TN = GemvTune<MODE>;
      return launch_variant<Q, MODE, TN::R, 1, false, true, TN::BLK>(a, stream, TN::PER_CU * kNumCUs);
    }
    return launch_t<Q, MODE, false, true>(a, stream);
  } else if constexpr (MODE == GM_QKV) {
    // Equal work per CU: when the rotation-pair units split evenly over the
    // CUs (7B: 2304 = 9 per CU, 14B: 3584 = 14), one block per CU with one
    // wave per unit.  The default 4 x 256-thread blocks per CU would give
    // 576 blocks for 7B, i.e. CUs with 2 and with 3 blocks, and the launch
    // would last as long as the CUs with 3.
    using TN = GemvTune<MODE>;
    const int units = units_total<MODE, TN::R>(a);
    if (norm && units % kNumCUs == 0) {
      if (units / kNumCUs == 9) return launch_variant<Q, MODE, TN::R, TN::U, true, true, 9 * kWave>(a, stream, kNumCUs);
      if (units / kNumCUs == 14) return launch_variant<Q, MODE, TN::R, TN::U, true, true, 14 * kWave>(a, stream, kNumCUs);
    }
    return norm ? launch_t<Q, MODE, true, true>(a, stream) : launch_t<Q, MODE, false, true>(a, stream);
  } else {
    if constexpr (MODE == GM_SWIGLU) {
      if (a.x_acc) {
        using TN = GemvTune<MODE>;
        return launch_variant<Q, MODE, TN::R, TN::U, true, true, TN::BLK, true>(a, stream, TN::PER_CU * kNumCUs);
      }
    }
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
