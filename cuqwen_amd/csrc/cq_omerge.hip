// Attention merge + O-projection in one launch, split over query heads.
//
// Reference: the split-K attention's stage 2 (src/kernels.cu:222-288) and the
// O-projection gemv_add (kernels.cu:640-687) are two dependent launches.
// Here block (head h, row band c) merges head h's stage-1 partials itself
// (the log-sum-exp rule of stage 2; the partials read as whole contiguous
// rows, each wave weighting its rows, the sums finished across lanes and
// waves), stages the fp16 attention output in LDS and multiplies it by the
// column slice Wo[band rows][h*hd .. (h+1)*hd), which
// the 128-column panel layout of Wo (wo_to_panels, below) makes one
// contiguous run of HBM.  The head contributions of an output row
// are summed in a 64-bit fixed-point accumulator (value * 2^32, one atomic
// add per row and head; integer adds are associative, so the result does
// not depend on arrival order and every run is bit-identical).  The next
// launch (RMSNorm + gate/up) turns accumulator + residual into the fp16
// residual stream, h = half(residual + sum) as in kernels.cu:671, and the
// down projection clears the accumulator for the next layer.
//
// What this saves is the stage-2 launch: on this part every dependent graph
// node costs about 1.6 us before its first wave runs, and the merge itself is
// latency-bound, so doing it in the projection's prologue -- while the
// projection's weights are already in flight -- hides most of it.
#include "cq_attention.h"
#include "cq_gemv.h"

#include <algorithm>

namespace cq {

constexpr int kOmDims = 16;                 // columns of the block's slice per wave
constexpr float kFixScale = 4294967296.f;   // 2^32
// |contribution| <= 2^20 (far beyond fp16's range: a row whose sum gets
// there ends as +-inf in fp16 either way) keeps the sum of up to 1024 heads
// below 2^62 in int64 and its integer part inside int32
constexpr float kFixClamp = 1048576.f;

// Row band of a block, blocks of one head placed XCD-major: workgroups are
// dealt round robin to the 8 XCDs (blockIdx % 8), so numbering them by
// (blockIdx % 8, blockIdx / 8) gives each XCD a contiguous run of heads and
// the blocks of one head mostly share their XCD's L2 copy of its partials.
__device__ __forceinline__ int om_order(int b, int nb) {
  const int x = b & 7, j = b >> 3;
  const int before = x * (nb >> 3) + min(x, nb & 7);   // blocks on XCDs 0..x-1
  return before + j;
}

// Q: weight format of Wo, HD: head dim, HPB: heads per block (the block
// covers one 128-column panel: two heads at head_dim 64), NR: rounds of row
// loads per wave.  One wave per 16 columns: 8 waves for a 128-column panel,
// 4 for a 64-column one.
// WM: 1, or 2 for twice the waves (bands of many rows: half the load rounds
// per wave).
template <int HD, int HPB, int WM>
struct OmShape {
  static constexpr int THREADS = HPB * HD / kOmDims * WM * kWave;
};

template <int Q, int HD, int HPB, int NR, int WM>
__global__ __launch_bounds__(HPB * HD / kOmDims * WM * kWave) void omerge_kernel(const OMergeArgs a) {
  using T = QTraits<Q>;
  CQ_PIN(gridDim.x); CQ_PIN(a.workspace); CQ_PIN(a.attn); CQ_PIN(a.W); CQ_PIN(a.acc); CQ_PIN(a.d_pos);
  CQ_PIN(a.n_heads); CQ_PIN(a.n_kv); CQ_PIN(a.K); CQ_PIN(a.N); CQ_PIN(a.Pmax); CQ_PIN(a.bands); CQ_PIN((int)a.direct);
  if constexpr (Q != CQ_QUANT_FP16) CQ_PIN(a.S);
  constexpr int W = HPB * HD;               // columns of the block's slice
  constexpr int WAVES = W / kOmDims * WM;
  constexpr int NCH = W / T::EPC;           // 16-byte chunks of one row slice
  constexpr int RPW = kWave / NCH;          // rows per wave per round
  constexpr int RPR = WAVES * RPW;          // rows per block per round
  constexpr int LPR = HD / 4;               // lanes per partition row (16 bytes each)
  constexpr int RPI = kWave / LPR;          // partition rows per wave instruction
  constexpr int NI = kWave / (WAVES * RPI); // instructions per wave per head and 64 partitions
  static_assert(NCH >= 1 && NCH <= kWave, "omerge: head_dim / format");
  static_assert(NI >= 1 && NI * WAVES * RPI == kWave, "omerge: merge tiling");
  __shared__ __align__(16) _Float16 attn[W];
  __shared__ __align__(16) float part[WAVES][W];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  // Unsigned 32-bit index arithmetic throughout (every offset here is far
  // below 2^31, host-checked): the prologue's address math runs on the CU's
  // one scalar unit for every resident wave, and signed or 64-bit division
  // and multiplication cost it several times the instructions.
  const uint32_t g = om_order(blockIdx.x, gridDim.x);
  const uint32_t bands = (uint32_t)a.bands, N = (uint32_t)a.N, Pmax = (uint32_t)a.Pmax;
  const int hq0 = (int)(g / bands) * HPB, band = (int)(g % bands);
  const int row0 = (int)(((uint32_t)band * N) / bands);
  const int row1 = (int)(((uint32_t)(band + 1) * N) / bands);
  const uint32_t gsz = (uint32_t)(a.n_heads / a.n_kv);

  // 1. the first 64 partitions of the block's heads, read coalesced: the
  //    partials are head-major (a head's partitions are contiguous 512-byte
  //    rows at head_dim 128), so one wave instruction covers RPI whole rows.
  //    (Lane-per-partition reads touched 64 cache lines per instruction and
  //    held the CU's memory pipeline -- and the weight loads queued behind
  //    them -- for microseconds.)  Independent of the position: rows past the
  //    partition count are weighted 0 below.
  const float* ws_m = reinterpret_cast<const float*>(a.workspace);
  const float* ws_l = ws_m + (uint32_t)a.n_kv * Pmax * 16u;
  const float* ws_o = ws_l + (uint32_t)a.n_kv * Pmax * 16u;
  auto head_base = [&](int j) {
    const uint32_t hq = (uint32_t)(hq0 + j);
    return ((hq / gsz) * 16u + hq % gsz) * Pmax;
  };
  const int rsub = lane / LPR, d4 = (lane % LPR) * 4;
  float mp[HPB], lp[HPB];
  f4_t ov[HPB][NI];
  auto load_chunk = [&](int p0) {
#pragma unroll
    for (int j = 0; j < HPB; ++j) {
      const uint32_t base = head_base(j);
      mp[j] = ws_m[base + (uint32_t)min(p0 + lane, a.Pmax - 1)];
      lp[j] = ws_l[base + (uint32_t)min(p0 + lane, a.Pmax - 1)];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int p = p0 + (i * WAVES + wave) * RPI + rsub;
        ov[j][i] = *reinterpret_cast<const f4_t*>(ws_o + (base + (uint32_t)min(p, a.Pmax - 1)) * HD + d4);
      }
    }
  };
  load_chunk(0);
  // the single-partition case finds the normalised output where stage 1 wrote it
  uint32_t direct = 0;
  const _Float16* xb = reinterpret_cast<const _Float16*>(a.attn) + (uint32_t)hq0 * HD;
  if (threadIdx.x < W / 2) direct = reinterpret_cast<const uint32_t*>(xb)[threadIdx.x];
  const int T_ = (int)load_ctl_u32(a.d_pos) + 1;

  // 2. the weight slice: round r, wave w, lane -> row row0 + r*RPR + w*RPW +
  //    lane/NCH, chunk lane%NCH; rows past the band re-read its last row
  //    (never used).  Wo is held in 128-column panels (wo_panels): panel p =
  //    [N rows][128 columns], so a band's slice is one contiguous run.
  constexpr int CP = kGroup / T::EPC;       // chunks of a panel row
  const int cch = lane % NCH;
  const int kc = hq0 * HD / T::EPC + cch;   // this lane's chunk within a row
  const int pan = kc / CP;
  const char* wbase = reinterpret_cast<const char*>(a.W) + ((uint32_t)pan * N * CP + kc % CP) * 16u;
  const _Float16* sbase = reinterpret_cast<const _Float16*>(a.S) + (uint32_t)pan * N;   // scales [panel][N]
  u4_t wv[NR];
  _Float16 sc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int row = min(row0 + r * RPR + wave * RPW + lane / NCH, row1 - 1);
    wv[r] = load_u4_stream(wbase + (uint32_t)row * (CP * 16u));
    if constexpr (Q != CQ_QUANT_FP16) sc[r] = sbase[row];
  }

  // 3. merge (kernels.cu:222-288, 1 / (L + 1e-9)): every wave forms the
  //    running max M and sum L of each head from its 64 m / l values (the
  //    same on every wave), weights its own rows, and the per-dimension sums
  //    are finished across the lanes of a row group and then across the
  //    waves in LDS
  int tpp;
  const int nparts = a.direct ? 1 : attn_nparts(T_, a.Pmax, &tpp);
  float L[HPB];
  if (nparts == 1) {
    if (threadIdx.x < W / 2) reinterpret_cast<uint32_t*>(attn)[threadIdx.x] = direct;
  } else {
    float M[HPB];
    f4_t acc4[HPB];
#pragma unroll
    for (int j = 0; j < HPB; ++j) {
      M[j] = -INFINITY;
      L[j] = 0.f;
      acc4[j] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
    auto merge_chunk = [&](int p0) {
#pragma unroll
      for (int j = 0; j < HPB; ++j) {
        const bool valid = p0 + lane < nparts && mp[j] != -INFINITY;
        const float Mn = fmaxf(M[j], wave_max(valid ? mp[j] : -INFINITY));
        const float f = M[j] == -INFINITY ? 0.f : __expf(M[j] - Mn);
        const float wgt = valid ? __expf(mp[j] - Mn) : 0.f;
        L[j] = L[j] * f + wave_sum(valid ? lp[j] * wgt : 0.f);
        f4_t s4 = acc4[j] * f;
#pragma unroll
        for (int i = 0; i < NI; ++i) s4 += ov[j][i] * __shfl(wgt, (i * WAVES + wave) * RPI + rsub, kWave);
        acc4[j] = s4;
        M[j] = Mn;
      }
    };
    // the first chunk straight from the registers loaded above (outside the
    // loop, so the wait for them leaves the weight loads in flight)
    merge_chunk(0);
    for (int p0 = kWave; p0 < nparts; p0 += kWave) {
      load_chunk(p0);
      merge_chunk(p0);
    }
#pragma unroll
    for (int j = 0; j < HPB; ++j) {
#pragma unroll
      for (int off = LPR; off < kWave; off <<= 1)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc4[j][e] += __shfl_xor(acc4[j][e], off, kWave);
      if (rsub == 0) *reinterpret_cast<f4_t*>(&part[wave][j * HD + d4]) = acc4[j];
    }
  }
  __syncthreads();
  if (nparts > 1 && threadIdx.x < W) {
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) o += part[w][threadIdx.x];
    const int j = threadIdx.x / HD;
    float lj = L[0];
#pragma unroll
    for (int jj = 1; jj < HPB; ++jj) lj = j == jj ? L[jj] : lj;
    attn[threadIdx.x] = (_Float16)(o * (1.0f / (lj + 1e-9f)));
  }
  __syncthreads();

  // 4. this lane's chunk of the heads' vector in the GEMV's plane order (plus
  //    the unpack-bias term), straight from LDS
  u4_t xv[T::PLANES];
  float corr = 0.f;
  {
    const u4_t* src = reinterpret_cast<const u4_t*>(attn) + cch * T::PLANES;
#pragma unroll
    for (int p = 0; p < T::PLANES; ++p) corr += plane_order_packed<Q>(src[p], xv[p]);
  }

  // 5. row dots, reduced over the NCH lanes of a row, one atomic per row
  const UnpackRegs uk = unpack_regs();
  unsigned long long* acc = reinterpret_cast<unsigned long long*>(a.acc);
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float v = chunk_dot<Q>(wv[r], xv, uk);
    if constexpr (Q != CQ_QUANT_FP16) v = (v - corr) * (float)sc[r];
#pragma unroll
    for (int off = NCH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    const int row = row0 + r * RPR + wave * RPW + lane / NCH;
    if (cch == 0 && row < row1) {
      v = fminf(kFixClamp, fmaxf(-kFixClamp, v));
      const long long fx = __float2ll_rn(v * kFixScale);
      atomicAdd(acc + row, (unsigned long long)fx);
    }
  }
}

template <int Q, int HD, int HPB>
static void omerge_launch_h(const OMergeArgs& a, hipStream_t stream, int nr, int wm, int blocks) {
  const dim3 grid(blocks);
  if (wm == 2) {
    const dim3 block(OmShape<HD, HPB, 2>::THREADS);
    // twice the waves only when one wave set needed more than 4 rounds: 4 or 8 remain
    if (nr <= 4) hipLaunchKernelGGL((omerge_kernel<Q, HD, HPB, 4, 2>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((omerge_kernel<Q, HD, HPB, 8, 2>), grid, block, 0, stream, a);
    return;
  }
  const dim3 block(OmShape<HD, HPB, 1>::THREADS);
  switch (nr) {
    case 1: hipLaunchKernelGGL((omerge_kernel<Q, HD, HPB, 1, 1>), grid, block, 0, stream, a); break;
    case 2: hipLaunchKernelGGL((omerge_kernel<Q, HD, HPB, 2, 1>), grid, block, 0, stream, a); break;
    case 4: hipLaunchKernelGGL((omerge_kernel<Q, HD, HPB, 4, 1>), grid, block, 0, stream, a); break;
    case 8: hipLaunchKernelGGL((omerge_kernel<Q, HD, HPB, 8, 1>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((omerge_kernel<Q, HD, HPB, 16, 1>), grid, block, 0, stream, a); break;
  }
}

// head_dim 64 always pairs heads (the config check makes n_heads * 64 a
// multiple of 128, so the head count is even)
template <int Q, int HD>
static void omerge_launch_q(const OMergeArgs& a, hipStream_t stream, int nr, int wm, int blocks) {
  omerge_launch_h<Q, HD, HD == 64 ? 2 : 1>(a, stream, nr, wm, blocks);
}

// ------------------------------------------- short contexts: attention + O-projection
// When a kv head's whole context is short, its attention is cheap enough to
// compute in every block that needs it, and the split over partitions (and
// the launch boundary between stage 1 and the merge) can go.  Block (kv head
// k, row band c) runs stage 1's tile loop over all T keys with its 8 waves
// (wave w takes tiles w, w + 8, ...), merges the waves in LDS into the
// group's normalised attention output -- exactly what a single-partition
// stage 1 writes -- and multiplies it by Wo[band rows][group columns]: the
// g heads of the group are g * hd contiguous columns of Wo, read here as
// 16-byte chunks through the 128-column panel layout.  One fixed-point
// atomic per row and kv head into the same accumulator as omerge_kernel,
// so the MLP launch that follows is unchanged.
//
// Lanes of a row: the group's chunks per row padded to a power of two P2,
// CPL chunks per lane (P2 / CPL <= 64 lanes), rows per wave 64 / (P2 / CPL);
// NR rounds of rows per wave, all requested before the attention starts.
template <int Q, int HD, int NR, int CPL>
__global__ __launch_bounds__(kAttnThreads) void attn_oproj_kernel(const AttnArgs at, const OMergeArgs a) {
  using T = QTraits<Q>;
  pin_attn_args<false>(at);
  CQ_PIN(a.W); CQ_PIN(a.acc); CQ_PIN(a.N); CQ_PIN(a.bands);
  if constexpr (Q != CQ_QUANT_FP16) CQ_PIN(a.S);
  constexpr int KK = HD / 32, DT = HD / 16;
  constexpr int CP = kGroup / T::EPC;   // chunks of a panel row
  __shared__ __align__(16) _Float16 attn_s[16 * HD];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t gi = om_order(blockIdx.x, gridDim.x);   // a kv head's bands share an XCD's L2 copy of its K/V
  const uint32_t bands = (uint32_t)a.bands, N = (uint32_t)a.N;
  const int kvh = (int)(gi / bands), band = (int)(gi % bands);
  const int row0 = (int)(((uint32_t)band * N) / bands);
  const int row1 = (int)(((uint32_t)(band + 1) * N) / bands);
  const int g = at.n_heads / at.n_kv;
  const int Tn = (int)load_ctl_u32(at.d_pos) + 1;
  const int n_tiles = (Tn + kTileKeys - 1) / kTileKeys;

  // 1. the wave's first K/V tile, then q of the group (stage 1's order)
  const _Float16* kbase = reinterpret_cast<const _Float16*>(at.kcache) + (int64_t)kvh * at.max_seq * HD;
  const _Float16* vbase = reinterpret_cast<const _Float16*>(at.vcache) + (int64_t)kvh * at.max_seq * HD;
  const KVRes kv{kbase, vbase, at.max_seq * HD * 2};
  KVTile<HD> A, B;
  int ti = wave;
  load_tile<HD>(A, kv, ti, ti < n_tiles, lane);
  const int h = lane & 15, j = lane >> 4;
  h8_t qb[KK];
  {
    const _Float16* q = reinterpret_cast<const _Float16*>(at.q) + (int64_t)(kvh * g + h) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (h < g) qb[kk] = __builtin_bit_cast(h8_t, load_u4(q + kk * 32 + j * 8));
      else qb[kk] = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  // 2. the band's weight slice (consumed after the attention)
  const int nchg = g * HD / T::EPC;   // chunks of the group's columns in one row
  int p2 = 1;
  while (p2 < nchg) p2 <<= 1;
  const int lpr = p2 / CPL;           // lanes per row (host-checked <= 64)
  const int rpw = kWave / lpr, rpr = kAttnWaves * rpw;
  const int lrow = lane / lpr, cl = lane % lpr;
  u4_t wv[NR][CPL];
  _Float16 sc[NR][CPL];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const uint32_t row = (uint32_t)min(row0 + r * rpr + wave * rpw + lrow, row1 - 1);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = cl + c * lpr;
      wv[r][c] = u4_t{0u, 0u, 0u, 0u};
      sc[r][c] = (_Float16)0.f;
      if (ch < nchg) {
        const uint32_t kc = (uint32_t)(kvh * nchg + ch), pan = kc / CP;
        wv[r][c] = load_u4_stream(reinterpret_cast<const char*>(a.W) + ((pan * N + row) * CP + kc % CP) * 16u);
        if constexpr (Q != CQ_QUANT_FP16) sc[r][c] = reinterpret_cast<const _Float16*>(a.S)[pan * N + row];
      }
    }
  }

  // 3. the whole context, then the 8-wave merge into the normalised output
  float m = -INFINITY, l = 0.f;
  f4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  attend_partition<HD>(A, B, qb, ti, n_tiles, Tn, kv, lane, m, l, o);
  block_merge_store<HD>(kvh, 0, g, m, l, o, nullptr, nullptr, nullptr, 0, attn_s);
  __syncthreads();

  // 4. the lane's chunks of the group's output in the GEMV's plane order
  u4_t xv[CPL][T::PLANES];
  float corr[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = cl + c * lpr;
    corr[c] = 0.f;
    if (ch < nchg) {
      const u4_t* src = reinterpret_cast<const u4_t*>(attn_s) + ch * T::PLANES;
#pragma unroll
      for (int p = 0; p < T::PLANES; ++p) corr[c] += plane_order_packed<Q>(src[p], xv[c][p]);
    } else {
#pragma unroll
      for (int p = 0; p < T::PLANES; ++p) xv[c][p] = u4_t{0u, 0u, 0u, 0u};
    }
  }

  // 5. row dots, reduced over the row's lanes, one atomic per row
  const UnpackRegs uk = unpack_regs();
  unsigned long long* acc = reinterpret_cast<unsigned long long*>(a.acc);
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float v = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const float d = chunk_dot<Q>(wv[r][c], xv[c], uk);
      if constexpr (Q != CQ_QUANT_FP16) v = fmaf(d - corr[c], (float)sc[r][c], v);
      else v += d;
    }
    for (int off = lpr / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    const int row = row0 + r * rpr + wave * rpw + lrow;
    if (cl == 0 && row < row1) {
      v = fminf(kFixClamp, fmaxf(-kFixClamp, v));
      const long long fx = __float2ll_rn(v * kFixScale);
      atomicAdd(acc + row, (unsigned long long)fx);
    }
  }
}

int attn_oproj_plan(int quant, int head_dim, int n_heads, int n_kv, int N, int* bands, int* rounds, int* cpl) {
  const int epc = quant == CQ_QUANT_INT4 ? 32 : quant == CQ_QUANT_INT8 ? 16 : 8;
  const int nchg = n_heads / n_kv * head_dim / epc;
  int p2 = 1;
  while (p2 < nchg) p2 <<= 1;
  const int c = p2 > kWave ? p2 / kWave : 1;
  if (c > 2) return fail(CQ_EINVAL, "attention + O-projection: group too wide");
  const int rpr = kAttnWaves * (kWave / (p2 / c));
  // rounds of rows per wave that fit the registers beside the attention's
  // (head_dim 128: NR * CPL <= 4, head_dim 64: NR <= 8)
  const int max_nr = head_dim == 128 ? 4 / c : 8;
  int b = std::max(1, kNumCUs / n_kv);
  b = std::max(b, (N + max_nr * rpr - 1) / (max_nr * rpr));
  b = std::min(b, N);
  const int rows = (N + b - 1) / b;
  const int nr = (rows + rpr - 1) / rpr;
  int r2 = 1;
  while (r2 < nr) r2 <<= 1;
  *bands = b;
  *rounds = r2;
  *cpl = c;
  return CQ_OK;
}

template <int Q, int HD, int CPL>
static void attn_oproj_launch_c(const AttnArgs& at, const OMergeArgs& a, int nr, hipStream_t stream) {
  const dim3 grid(a.n_kv * a.bands), block(kAttnThreads);
  switch (nr) {
    case 1: hipLaunchKernelGGL((attn_oproj_kernel<Q, HD, 1, CPL>), grid, block, 0, stream, at, a); break;
    case 2: hipLaunchKernelGGL((attn_oproj_kernel<Q, HD, 2, CPL>), grid, block, 0, stream, at, a); break;
    case 4: hipLaunchKernelGGL((attn_oproj_kernel<Q, HD, 4, CPL>), grid, block, 0, stream, at, a); break;
    default: hipLaunchKernelGGL((attn_oproj_kernel<Q, HD, 8, CPL>), grid, block, 0, stream, at, a); break;
  }
}

template <int Q, int HD>
static void attn_oproj_launch_q(const AttnArgs& at, const OMergeArgs& a, int nr, int cpl, hipStream_t stream) {
  if (cpl == 2) attn_oproj_launch_c<Q, HD, 2>(at, a, nr, stream);
  else attn_oproj_launch_c<Q, HD, 1>(at, a, nr, stream);
}

int launch_attn_oproj(const AttnArgs& at, const OMergeArgs& a0, hipStream_t stream) {
  OMergeArgs a = a0;
  if (!at.kcache || !at.vcache || at.kcache8) return fail(CQ_EINVAL, "attention + O-projection: fp16 cache only");
  if (a.head_dim != 64 && a.head_dim != 128) return fail(CQ_EINVAL, "attention + O-projection: head_dim must be 64 or 128");
  if (a.quant < 0 || a.quant > 2) return fail(CQ_EINVAL, "attention + O-projection: bad quant type");
  if (a.n_kv <= 0 || a.n_heads % a.n_kv || a.n_heads / a.n_kv > 16) return fail(CQ_EINVAL, "attention + O-projection: bad head layout");
  if (a.K != a.n_heads * a.head_dim || a.N <= 0 || a.K % kGroup) return fail(CQ_EINVAL, "attention + O-projection: bad shape");
  if (at.n_heads != a.n_heads || at.n_kv != a.n_kv || at.head_dim != a.head_dim || at.d_pos != a.d_pos)
    return fail(CQ_EINVAL, "attention + O-projection: attention and projection shapes differ");
  if (!at.q || !a.W || !a.acc || !a.d_pos || (a.quant != CQ_QUANT_FP16 && !a.S))
    return fail(CQ_EINVAL, "attention + O-projection: null pointer");
  int nr = 1, cpl = 1;
  CQ_TRY(attn_oproj_plan(a.quant, a.head_dim, a.n_heads, a.n_kv, a.N, &a.bands, &nr, &cpl));
  if ((int64_t)a.N * a.K * 2 >= ((int64_t)1 << 31) || (int64_t)a.N * (a.bands + 1) >= ((int64_t)1 << 31) ||
      (int64_t)at.max_seq * a.head_dim * 2 >= ((int64_t)1 << 31))
    return fail(CQ_EINVAL, "attention + O-projection: shape too large for 32-bit indexing");
  if (a.quant == CQ_QUANT_INT4) {
    if (a.head_dim == 128) attn_oproj_launch_q<CQ_QUANT_INT4, 128>(at, a, nr, cpl, stream);
    else attn_oproj_launch_q<CQ_QUANT_INT4, 64>(at, a, nr, cpl, stream);
  } else if (a.quant == CQ_QUANT_INT8) {
    if (a.head_dim == 128) attn_oproj_launch_q<CQ_QUANT_INT8, 128>(at, a, nr, cpl, stream);
    else attn_oproj_launch_q<CQ_QUANT_INT8, 64>(at, a, nr, cpl, stream);
  } else {
    if (a.head_dim == 128) attn_oproj_launch_q<CQ_QUANT_FP16, 128>(at, a, nr, cpl, stream);
    else attn_oproj_launch_q<CQ_QUANT_FP16, 64>(at, a, nr, cpl, stream);
  }
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

// ------------------------------------------------------------ Wo panels
// Row-major [N][K] (the file's layout) -> K/128 panels of [N][128]: 16-byte
// chunk c of row n (chunk c % CP of panel c / CP) moves to
// ((c / CP) * N + n) * CP + c % CP; group-128 scales [N][K/128] -> [K/128][N].
__global__ void panelize_kernel(const u4_t* src, u4_t* dst, int N, int NC, int CP) {
  const int64_t total = (int64_t)N * NC;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(i / NC), c = (int)(i % NC);
    dst[((int64_t)(c / CP) * N + n) * CP + c % CP] = src[i];
  }
}
__global__ void panelize_scales_kernel(const uint16_t* src, uint16_t* dst, int N, int G) {
  const int64_t total = (int64_t)N * G;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(i / G), g = (int)(i % G);
    dst[(int64_t)g * N + n] = src[i];
  }
}

// The inverse of the two above: panels -> row-major [N][K], scales
// [K/128][N] -> [N][K/128] (the exporter's layouts), out of place.
__global__ void unpanelize_kernel(const u4_t* src, u4_t* dst, int N, int NC, int CP) {
  const int64_t total = (int64_t)N * NC;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(i / NC), c = (int)(i % NC);
    dst[i] = src[((int64_t)(c / CP) * N + n) * CP + c % CP];
  }
}
__global__ void unpanelize_scales_kernel(const uint16_t* src, uint16_t* dst, int N, int G) {
  const int64_t total = (int64_t)N * G;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(i / G), g = (int)(i % G);
    dst[i] = src[(int64_t)g * N + n];
  }
}

int wo_from_panels(int quant, const void* W, const __half* S, int N, int K, void* W_rows, __half* S_rows,
                   hipStream_t stream) {
  if (K % kGroup) return fail(CQ_EINVAL, "wo rows: K must be a multiple of 128");
  const int epc = quant == CQ_QUANT_INT4 ? 32 : quant == CQ_QUANT_INT8 ? 16 : 8;
  const int NC = K / epc, CP = kGroup / epc;
  hipLaunchKernelGGL(unpanelize_kernel, dim3(1024), dim3(256), 0, stream, (const u4_t*)W, (u4_t*)W_rows, N, NC, CP);
  CQ_HIP(hipGetLastError());
  if (quant != CQ_QUANT_FP16) {
    hipLaunchKernelGGL(unpanelize_scales_kernel, dim3(256), dim3(256), 0, stream, (const uint16_t*)S,
                       (uint16_t*)S_rows, N, K / kGroup);
    CQ_HIP(hipGetLastError());
  }
  return CQ_OK;
}

int wo_to_panels(int quant, void* W, __half* S, int N, int K, void* tmp, hipStream_t stream) {
  if (K % kGroup) return fail(CQ_EINVAL, "wo panels: K must be a multiple of 128");
  const int epc = quant == CQ_QUANT_INT4 ? 32 : quant == CQ_QUANT_INT8 ? 16 : 8;
  const int NC = K / epc, CP = kGroup / epc;
  const size_t wbytes = (size_t)N * NC * 16;
  hipLaunchKernelGGL(panelize_kernel, dim3(1024), dim3(256), 0, stream, (const u4_t*)W, (u4_t*)tmp, N, NC, CP);
  CQ_HIP(hipGetLastError());
  CQ_HIP(hipMemcpyAsync(W, tmp, wbytes, hipMemcpyDeviceToDevice, stream));
  if (quant != CQ_QUANT_FP16) {
    const int G = K / kGroup;
    hipLaunchKernelGGL(panelize_scales_kernel, dim3(256), dim3(256), 0, stream, (const uint16_t*)S, (uint16_t*)tmp, N, G);
    CQ_HIP(hipGetLastError());
    CQ_HIP(hipMemcpyAsync(S, tmp, (size_t)N * G * 2, hipMemcpyDeviceToDevice, stream));
  }
  return CQ_OK;
}

// Heads per block: one 128-column panel (two heads at head_dim 64).  Bands per head group: as many as fit one block per
// CU (7B: 28 heads x 9 bands = 252 blocks), more when a band would need more
// than 16 rounds of row loads, twice as many when a band would exceed 512 rows.  Bands that need more than 4 rounds with the
// base wave count (int8 / fp16 at 7B, 14B) run twice the waves.
int omerge_plan(int quant, int head_dim, int n_heads, int N, int* hpb, int* bands, int* rounds, int* wm) {
  const int epc = quant == CQ_QUANT_INT4 ? 32 : quant == CQ_QUANT_INT8 ? 16 : 8;
  const int h = head_dim == 64 ? 2 : 1;
  const int nch = h * head_dim / epc;
  const int rpr1 = (h * head_dim / kOmDims) * (kWave / nch);
  const int groups = n_heads / h;
  int b = std::max(1, kNumCUs / groups);
  b = std::max(b, (N + 16 * rpr1 - 1) / (16 * rpr1));
  // long bands (14B: 853 rows) in two launch rounds of half the rows each:
  // 7.75 -> 7.2 us per launch measured (7B's 399-row bands are faster as one round)
  if ((N + b - 1) / b > 512) b *= 2;
  b = std::min(b, N);
  const int rows = (N + b - 1) / b;
  int w = (rows + rpr1 - 1) / rpr1 > 4 ? 2 : 1;
  const int nr = (rows + w * rpr1 - 1) / (w * rpr1);
  int p2 = 1;
  while (p2 < nr) p2 <<= 1;
  *hpb = h;
  *bands = b;
  *rounds = p2;
  *wm = w;
  return CQ_OK;
}

int launch_omerge(const OMergeArgs& a0, hipStream_t stream) {
  OMergeArgs a = a0;
  if (a.head_dim != 64 && a.head_dim != 128) return fail(CQ_EINVAL, "omerge: head_dim must be 64 or 128");
  if (a.quant < 0 || a.quant > 2) return fail(CQ_EINVAL, "omerge: bad quant type");
  if (a.n_kv <= 0 || a.n_heads % a.n_kv || a.n_heads / a.n_kv > 16) return fail(CQ_EINVAL, "omerge: bad head layout");
  if (a.K != a.n_heads * a.head_dim || a.N <= 0 || a.K % kGroup) return fail(CQ_EINVAL, "omerge: bad shape");
  if (!a.workspace || !a.attn || !a.W || !a.acc || !a.d_pos || (a.quant != CQ_QUANT_FP16 && !a.S))
    return fail(CQ_EINVAL, "omerge: null pointer");
  if (a.Pmax <= 0) return fail(CQ_EINVAL, "omerge: bad partition count");
  int hpb = 1, nr = 1, wm = 1;
  omerge_plan(a.quant, a.head_dim, a.n_heads, a.N, &hpb, &a.bands, &nr, &wm);
  // the kernel indexes in unsigned 32 bits: Wo bytes, the partial slots and
  // the band rows (with the band count the launch uses)
  if ((int64_t)a.N * a.K * 2 >= ((int64_t)1 << 31) || (int64_t)a.n_kv * 16 * a.Pmax * a.head_dim >= ((int64_t)1 << 31) ||
      (int64_t)a.N * (a.bands + 1) >= ((int64_t)1 << 31))
    return fail(CQ_EINVAL, "omerge: shape too large for 32-bit indexing");
  const int blocks = a.n_heads / hpb * a.bands;
  if (a.quant == CQ_QUANT_INT4) {
    if (a.head_dim == 128) omerge_launch_q<CQ_QUANT_INT4, 128>(a, stream, nr, wm, blocks);
    else omerge_launch_q<CQ_QUANT_INT4, 64>(a, stream, nr, wm, blocks);
  } else if (a.quant == CQ_QUANT_INT8) {
    if (a.head_dim == 128) omerge_launch_q<CQ_QUANT_INT8, 128>(a, stream, nr, wm, blocks);
    else omerge_launch_q<CQ_QUANT_INT8, 64>(a, stream, nr, wm, blocks);
  } else {
    if (a.head_dim == 128) omerge_launch_q<CQ_QUANT_FP16, 128>(a, stream, nr, wm, blocks);
    else omerge_launch_q<CQ_QUANT_FP16, 64>(a, stream, nr, wm, blocks);
  }
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

}  // namespace cq
