// Batched prefill for gfx950: the prompt goes through the layers M tokens at
// a time instead of one decode step per token (the reference's prefill loop,
// src/main.cu:87-92, calls qwen_forward once per prompt token; batched
// prefill is its roadmap item, README.md:145).
//
// Per layer and chunk of M tokens:
//   RMSNorm         x -> half(x * w) and rsqrt(mean(x^2) + eps) per token
//                   (the decode GEMVs' fused RMSNorm, kernels.cu:689-751):
//                   pf_norm_rows for layer 0, later in the epilogue of the
//                   residual GEMM that produces x
//   pf_gemm<QKV>    Q / K / V rows, bias, RoPE at each token's position, K / V
//                   into the cache (kernels.cu:402-474, :370-398, :326-347)
//   pf_attention    causal FlashDecoding over the cache (kernels.cu:105-288
//                   with a per-token key limit)
//   pf_gemm<RESID>  O-proj + residual (kernels.cu:640-687), + RMSNorm
//   pf_gemm<SWIGLU> (kernels.cu:523-585), pf_gemm<RESID> (down), + RMSNorm
// The GEMMs are M > 1, so they run on the matrix cores: each wave dequantizes
// its weight rows in registers (int4 / int8 to exact small-integer fp16,
// times the group's fp16 scale) as the A operand of v_mfma_f32_16x16x32_f16
// and takes 16-token slices of the activation tile, staged in LDS, as the B
// operand.
//
// Activation layout: the inputs of the GEMMs (normed x, attention output,
// SwiGLU output) are stored in the order in which the weights' unpack yields
// pairs (int4: each 8-group as [0,4,1,5,2,6,3,7] with the odd elements / 16;
// int8 / fp16: natural), so neither operand needs a shuffle in the main loop.
#include "cq_attention.h"
#include "cq_gemv.h"

#include <algorithm>
#include <type_traits>

namespace cq {

constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * 64;
constexpr int kPfK = 128;         // K per main-loop step (one quantization group)
constexpr int kPfMaxSplit = 8;

// Activation layout of the GEMM inputs, chosen by the weights' format so the
// A operand needs no shuffle: int4 stores each 8-group in the order
// [0,4,1,5,2,6,3,7] with the odd elements divided by 16 (the unpack yields the
// odd nibbles as 16 n without a shift); int8 and fp16 keep natural order.
__device__ __forceinline__ int pf_pos(int k, bool int4) {
  if (!int4) return k;
  const int e = k & 7;
  return (k & ~7) | (e < 4 ? 2 * e : 2 * e - 7);
}
// value stored for element k.  The /16 is a power-of-two scale, exact for
// |v| >= 2^-10; below that v/16 falls in fp16's subnormal range and keeps
// fewer bits (at most 2^-21 absolute error on the element: half the 2^-24
// subnormal spacing, times 16).
__device__ __forceinline__ _Float16 pf_val(float v, int k, bool int4) {
  return (_Float16)((int4 && (k & 1)) ? v * 0.0625f : v);
}

// ------------------------------------------------------------- row norm
// RMSNorm of one token row by one block (dim a multiple of 8): A row =
// half(x * w) in the layout of the weights' format, inv = rsqrt(mean(x^2) +
// half(eps)).  Without w, A = x (in the layout) and no inv.  Thread t takes
// the 8-element groups t, t + blockDim.x, ... (the layout permutes within a
// group, so each group is one 16-byte load and one 16-byte store).
__device__ __forceinline__ void pf_norm_row(const _Float16* xr, const _Float16* w, float eps, int dim, _Float16* ar,
                                            float* inv_m, bool int4, float* red) {
  float ss = 0.f;
  for (int g = threadIdx.x; g < dim / 8; g += blockDim.x) {
    const h8_t xv = __builtin_bit_cast(h8_t, load_u4(xr + 8 * g));
    h8_t wv;
    if (w) wv = __builtin_bit_cast(h8_t, load_u4(w + 8 * g));
    h8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = (float)xv[e];
      ss = fmaf(v, v, ss);
      // half(x * w) first (the decode GEMVs' staging), then the layout's scale
      const float y = w ? (float)(_Float16)(v * (float)wv[e]) : v;
      o[pf_pos(e, int4)] = pf_val(y, e, int4);
    }
    *reinterpret_cast<u4_t*>(ar + 8 * g) = __builtin_bit_cast(u4_t, o);
  }
  if (w) {
    ss = block_sum(ss, red);
    if (threadIdx.x == 0) *inv_m = rsqrtf(ss / (float)dim + (float)(_Float16)eps);
  }
}

// One block per token row.
__global__ __launch_bounds__(256) void pf_norm_rows(const _Float16* x, const _Float16* w, float eps, int dim,
                                                    _Float16* A, float* inv, bool int4) {
  __shared__ float red[16];
  const int m = blockIdx.x;
  pf_norm_row(x + (int64_t)m * dim, w, eps, dim, A + (int64_t)m * dim, inv + m, int4, red);
}

// Embedding rows of the chunk's tokens (kernels.cu:85-103).
__global__ __launch_bounds__(256) void pf_embed(const u4_t* embed, const int* tokens, u4_t* x, int vec_dim) {
  const int m = blockIdx.x;
  const int64_t t = tokens[m];
  for (int i = threadIdx.x; i < vec_dim; i += blockDim.x) x[(int64_t)m * vec_dim + i] = embed[t * vec_dim + i];
}

// ------------------------------------------------------------------ GEMM
template <int Q> struct PfW;   // 16-byte weight loads per lane per 128-wide step
template <> struct PfW<CQ_QUANT_INT4> { static constexpr int LOADS = 1; };
template <> struct PfW<CQ_QUANT_INT8> { static constexpr int LOADS = 2; };
template <> struct PfW<CQ_QUANT_FP16> { static constexpr int LOADS = 4; };

// The A operand (8 fp16 weights in the order [0,4,1,5,2,6,3,7] of true k
// j*32 + s*8 + e) for sub-step s from the lane's loaded bytes.
template <int Q>
__device__ __forceinline__ h8_t pf_unpack(const u4_t* w, int s, uint32_t m_lo, uint32_t m_hi, uint32_t magic) {
  u4_t o;
  if constexpr (Q == CQ_QUANT_INT4) {
    // word s: nibbles e0..e7 of true k j*32 + s*8 + e; after ^0x88888888 each
    // is n = q + 8.  (1024 + n) - 1032 = q for e0 e4 e2 e6; the odd nibbles
    // stay in place: (1024 + 16 n) - 1152 = 16 q against activations / 16.
    const uint32_t f = w[0][s] ^ kInt4Flip, f8 = f >> 8;
    const h2_t blo = {(_Float16)-1032.f, (_Float16)-1032.f}, bhi = {(_Float16)-1152.f, (_Float16)-1152.f};
    o.x = as_u32(as_h2(and_or(f, m_lo, 0x64006400u)) + blo);    // (e0, e4)
    o.y = as_u32(as_h2(and_or(f, m_hi, 0x64006400u)) + bhi);    // (16 e1, 16 e5)
    o.z = as_u32(as_h2(and_or(f8, m_lo, 0x64006400u)) + blo);   // (e2, e6)
    o.w = as_u32(as_h2(and_or(f8, m_hi, 0x64006400u)) + bhi);   // (16 e3, 16 e7)
  } else if constexpr (Q == CQ_QUANT_INT8) {
    // bytes 8s..8s+7 in natural order: (1152 + q) pairs, minus 1152
    const uint32_t f0 = w[s >> 1][(s & 1) * 2] ^ kInt8Flip, f1 = w[s >> 1][(s & 1) * 2 + 1] ^ kInt8Flip;
    const h2_t b = {(_Float16)-kInt8Bias, (_Float16)-kInt8Bias};
    o.x = as_u32(as_h2(int8_pair(f0, magic, 0)) + b);
    o.y = as_u32(as_h2(int8_pair(f0, magic, 1)) + b);
    o.z = as_u32(as_h2(int8_pair(f1, magic, 0)) + b);
    o.w = as_u32(as_h2(int8_pair(f1, magic, 1)) + b);
  } else {
    o = w[s];   // fp16, natural order
  }
  return __builtin_bit_cast(h8_t, o);
}

// Row r of the concatenated output (QKV: q rows, then k, then v) -> matrix.
__device__ __forceinline__ int pf_mat(const PfGemmArgs& a, int row, int* local) {
  if (row < a.rows[0]) { *local = row; return 0; }
  if (row < a.rows[0] + a.rows[1]) { *local = row - a.rows[0]; return 1; }
  *local = row - a.rows[0] - a.rows[1];
  return 2;
}

// One rotated pair (rows local, local + hd/2 of matrix mat) of token m:
// q into the Q buffer, k / v into the cache at position pos0 + m.
__device__ __forceinline__ void pf_qkv_store(const PfGemmArgs& a, int mat, int local, int m, _Float16 h0, _Float16 h1) {
  const int hd = a.head_dim, half = hd / 2;
  if (mat == 0) {
    a.out[(int64_t)m * a.rows[0] + local] = h0;
    a.out[(int64_t)m * a.rows[0] + local + half] = h1;
  } else {
    const int kvh = local / hd, i = local % hd, pos = a.pos0 + m;
    _Float16* c = mat == 1 ? a.kcache : a.vcache;
    if (mat == 1) {
      c[kv_k_offset(kvh, pos, i, a.max_seq, hd)] = h0;
      c[kv_k_offset(kvh, pos, i + half, a.max_seq, hd)] = h1;
    } else {
      c[kv_v_offset(kvh, pos, i, a.max_seq, hd)] = h0;
      c[kv_v_offset(kvh, pos, i + half, a.max_seq, hd)] = h1;
    }
  }
}

// One (token, kv head) row into the quantized cache: s = max|x| / code max
// (a zero row keeps s = 0 and q = 0), q = code of x / s (int8: rint clamped
// to +-127; E4M3: round to nearest even); element d from value(d).
template <typename F>
__device__ __forceinline__ void pf_kv8_store(const PfGemmArgs& a, int mat, int kvh, int pos, float amax, F value) {
  const int hd = a.head_dim;
  const bool f8 = a.kv_fmt == CQ_KV_FP8;
  const float sc = amax / (f8 ? kv_code_max<CQ_KV_FP8>() : kv_code_max<CQ_KV_INT8>());
  int8_t* c = mat == 1 ? a.kcache8 : a.vcache8;
  for (int d = 0; d < hd; ++d) {
    const float v = value(d) / sc;
    const int8_t q = sc == 0.f ? (int8_t)0 : (f8 ? kv_encode<CQ_KV_FP8>(v) : kv_encode<CQ_KV_INT8>(v));
    c[mat == 1 ? kv8_k_offset(kvh, pos, d, a.max_seq, hd) : kv8_v_offset(kvh, pos, d, a.max_seq, hd)] = q;
  }
  (mat == 1 ? a.kscale : a.vscale)[(int64_t)kvh * a.max_seq + pos] = sc;
}

template <int Q>
__device__ __forceinline__ void pf_load_w(const PfGemmArgs& a, const char* rowp, int ks, int j, u4_t* w) {
  constexpr int L = PfW<Q>::LOADS;
  // 64*L bytes of the row per step (panels: one panel row, panel stride N rows), L*16 per lane
  const int64_t kstep = a.panels ? (int64_t)a.N * (64 * L) : 64 * L;
  const char* p = rowp + (int64_t)ks * kstep + j * (L * 16);
#pragma unroll
  for (int i = 0; i < L; ++i) w[i] = load_u4(p + i * 16);
}

// Tile shape: RT 16-row slices per wave (SwiGLU: RT/2 gate and RT/2 up
// slices of the same output rows), 8 token slices of 16 per wave (the unpack
// of a weight fragment is shared by 8 matrix instructions); a block is 8
// waves over the same 128 tokens, two per SIMD.
template <int Q> struct PfTile { static constexpr int RT = 2; };
constexpr int kPfTT = 8;                         // token slices per wave
constexpr int kPfTok = 16 * kPfTT;               // tokens per block
template <int Q, int MODE> struct PfShape {
  static constexpr int NMAT = MODE == GM_SWIGLU ? 2 : 1;
  static constexpr int RT = PfTile<Q>::RT / NMAT;   // row slices per matrix
  static constexpr int WROWS = RT * 16;              // output rows per wave
  static constexpr int BN = kPfWaves * WROWS;        // output rows per block
};

// The block's (row block, token block) from its dispatch index, so that all
// token blocks of a row block run on one XCD and share its weight rows in
// that XCD's L2: dispatch goes round-robin over the 8 XCDs, so XCD x runs
// blocks x, x + 8, ...; those take a contiguous range of row-major tiles.
__device__ __forceinline__ void pf_block_tile(int n_tb, int* rb, int* tb) {
  const int id = blockIdx.x, n = gridDim.x;
  const int xcd = id & 7, k = id >> 3, base = n >> 3, rem = n & 7;
  const int L = xcd * base + min(xcd, rem) + k;
  *rb = L / n_tb;
  *tb = L % n_tb;
}

// 16-byte slot of K chunk c (0..15) in activation row t of a GEMM LDS stage,
// and, the map being an involution, the chunk held in slot c.  A 16-byte LDS
// read on gfx950 serves each 32-lane half of a wave in two passes of 16
// lanes split by the parity of lane bits 2..4 (lanes 0-3, 12-15, 20-27 and
// 4-11, 16-19, 28-31; measured with per-lane-pair probes and
// SQ_LDS_BANK_CONFLICT); a pass takes one cycle when its 16 lanes hit 16
// different 16-byte bank groups of the 256-byte bank row.  The B read has
// lane (r, j) = (lane % 16, lane / 16) at row r, chunk 4j + s4: XOR with
// f(r) = r ^ 8 * (bit 2 of r ^ bit 3 of r) gives every pass 16 different
// slots, where XOR with r alone puts two lanes of each pass on one slot.
__device__ __forceinline__ int pf_slot(int t, int c) {
  const int r = t & 15;
  return c ^ r ^ ((((r >> 2) ^ (r >> 3)) & 1) << 3);
}

// C^T tile of a wave: NMAT matrices (SwiGLU: gate and up) x RT row slices of
// 16 x 8 token slices of 16; lane holds rows 4*(lane/16)+v, token lane%16.
// The group scale multiplies the unpacked weights (half(q * s), one packed
// multiply per pair), so the matrix cores accumulate the whole K range
// directly into the tile.
template <int Q, int MODE, bool SPLIT>
__global__ __launch_bounds__(kPfThreads, 2) void pf_gemm_kernel(const PfGemmArgs a) {
  using SH = PfShape<Q, MODE>;
  constexpr int NMAT = SH::NMAT, RT = SH::RT, WROWS = SH::WROWS, BN = SH::BN, TT = kPfTT;
  constexpr int L = PfW<Q>::LOADS;
  constexpr int XS = kPfTok * kPfK;                         // halves of one activation stage
  constexpr int OT = MODE == GM_QKV ? kPfTok / 2 * (BN + 2) : 0;   // QKV epilogue tile (half the tokens x rows)
  constexpr int NS = 2;                                     // LDS stages
  // the epilogues reuse the stages: QKV tile, residual fp32 half tile
  constexpr int SM = std::max({NS * XS, OT, kPfTok / 2 * (BN + 4) * 2});
  __shared__ __align__(16) _Float16 smem[SM];
  _Float16* xs0 = smem;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r = lane & 15, j = lane >> 4;
  const int n_tb = (a.M + kPfTok - 1) / kPfTok;
  int rb, tb;
  pf_block_tile(n_tb, &rb, &tb);
  const int m0 = tb * kPfTok;
  const int nb0 = rb * BN;                     // first output row of the block
  const int nw0 = nb0 + wave * WROWS;          // first output row of the wave
  const int K = a.K, nks = K / kPfK;
  // split-K: block z of gridDim.z sums K steps [kb, ke) into an fp32 partial
  const int kb = SPLIT ? (int)((int64_t)blockIdx.z * nks / gridDim.z) : 0;
  const int ke = SPLIT ? (int)((int64_t)(blockIdx.z + 1) * nks / gridDim.z) : nks;

  // weight row (A operand row r of each slice) and its scale row
  const int64_t sstep = a.panels ? a.N : 1;   // scale stride of one K step
  const char* rowp[NMAT][RT];
  const _Float16* srow[NMAT][RT];
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      int local, row = min(nw0 + rt * 16 + r, a.N - 1);
      const int mat = MODE == GM_SWIGLU ? mt : pf_mat(a, row, &local);
      if (MODE == GM_SWIGLU) local = row;
      // row-major: step ks is bytes [64*L*ks, 64*L*(ks+1)) of the row; panels: row
      // `local` of panel ks (wo_to_panels), scales [panel][N]
      const int64_t rbytes = a.panels ? 64 * L : Q == CQ_QUANT_INT4 ? K / 2 : Q == CQ_QUANT_INT8 ? K : 2 * K;
      rowp[mt][rt] = reinterpret_cast<const char*>(sel3(a.W, mat)) + (int64_t)local * rbytes;
      srow[mt][rt] = Q == CQ_QUANT_FP16 ? nullptr : sel3(a.S, mat) + (a.panels ? (int64_t)local : (int64_t)local * (K / kGroup));
    }

  // Activation tiles: global -> registers one step ahead, then 16-byte LDS
  // stores into one of two stages at the start of the step that reads them
  // (measured faster than global_load_lds straight into LDS).  A stage holds
  // 128 token rows of 256 bytes; 16-byte slot s of row t holds K chunk
  // pf_slot(t, s) (an involution), so the B-operand reads are free of bank
  // conflicts.  Piece q of a step (q = i * waves + wave) is rows
  // 4q .. 4q + 3: lane l holds row 4q + l / 16, slot l % 16.
  constexpr int XL = kPfTok / (4 * kPfWaves);
  u4_t xr[XL];
  auto x_load = [&](int ks) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int q = i * kPfWaves + wave, t = 4 * q + (lane >> 4), c = pf_slot(t, lane & 15);
      const int m = min(m0 + t, a.M - 1);
      xr[i] = load_u4(a.A + (int64_t)m * K + ks * kPfK + c * 8);
    }
  };
  auto x_store = [&](int stg) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int q = i * kPfWaves + wave;
      *reinterpret_cast<u4_t*>(xs0 + stg * XS + q * 512 + lane * 8) = xr[i];
    }
  };
  f4_t acc[NMAT][RT][TT];
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[mt][rt][tt] = f4_t{0.f, 0.f, 0.f, 0.f};

  // Pipeline: at step k (after its barrier) the activations of step k+1
  // (into registers) and then the weights of step k+2 (into register set
  // k % 2) are requested; the K loop is unrolled by two so the weight
  // register sets keep compile-time indices.  At the start of step k a wave
  // waits until only the WL weight / scale loads of step k+1 are
  // outstanding, stores its piece of step k's activations into LDS stage
  // k % 2 (last read in step k-2, which every wave finished before step
  // k-1's barrier) and waits for the stores; the barrier then makes all
  // pieces visible.
  constexpr int WL = NMAT * RT * (L + (Q != CQ_QUANT_FP16 ? 1 : 0));
  static_assert(WL < 64, "vmcnt range");
  u4_t wv[2][NMAT][RT][L];
  _Float16 sv[2][NMAT][RT];
  auto load_w_step = [&](int ks, u4_t (&w)[NMAT][RT][L], _Float16 (&s)[NMAT][RT]) {
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        pf_load_w<Q>(a, rowp[mt][rt], ks, j, w[mt][rt]);
        if constexpr (Q != CQ_QUANT_FP16) s[mt][rt] = srow[mt][rt][(int64_t)ks * sstep];
      }
  };
  // Every load is issued unconditionally (step indices clamped to the last
  // step; the repeats past it are never used): with loads under branches the
  // compiler's wait-count tracking merges the paths conservatively and waits
  // for all loads, the next step's weight prefetch included, before the
  // activation stores of every step.
  load_w_step(kb, wv[0], sv[0]);
  x_load(kb);
  __builtin_amdgcn_sched_barrier(0);
  load_w_step(min(kb + 1, ke - 1), wv[1], sv[1]);

  const UnpackRegs uk = unpack_regs();
  auto step = [&](auto I, int ks) {
    constexpr int S = decltype(I)::value;   // weight register set of this step
    const int stg = (ks - kb) & 1;
    // simm16 of s_waitcnt on gfx9: vmcnt in bits [3:0] and [15:14], expcnt
    // [6:4], lgkmcnt [11:8]; the fields not waited on are left at their maxima
    __builtin_amdgcn_s_waitcnt(0x0F70 | (WL & 15) | ((WL >> 4) << 14));
    x_store(stg);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the LDS stores are done
    lds_barrier();
    const _Float16* xb0 = xs0 + stg * XS;
    h2_t s2[NMAT][RT];
    u4_t w[NMAT][RT][L];
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        s2[mt][rt] = h2_t{sv[S][mt][rt], sv[S][mt][rt]};
#pragma unroll
        for (int i = 0; i < L; ++i) w[mt][rt][i] = wv[S][mt][rt][i];
      }
    // activations first: the next step waits for them with the weights
    // requested here still in flight (the wait counts loads in issue order)
    x_load(min(ks + 1, ke - 1));
    __builtin_amdgcn_sched_barrier(0);
    load_w_step(min(ks + 2, ke - 1), wv[S], sv[S]);
    // B fragments of one sub-step
    auto read_b = [&](int s4, h8_t* xb) {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)   // row tt*16 + r, K chunk 4j + s4 at slot pf_slot(r, 4j + s4)
        xb[tt] = *reinterpret_cast<const h8_t*>(&xb0[(tt * 16 + r) * kPfK + pf_slot(r, 4 * j + s4) * 8]);
    };
    // A fragments (dequantized weights) of sub-step s4
    auto unpack_a = [&](int s4, h8_t (&wa)[NMAT][RT]) {
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          h8_t u = pf_unpack<Q>(w[mt][rt], s4, uk.m_lo, uk.m_hi, uk.magic);
          if constexpr (Q != CQ_QUANT_FP16) {
            u4_t uu = __builtin_bit_cast(u4_t, u);
            uu.x = as_u32(as_h2(uu.x) * s2[mt][rt]);
            uu.y = as_u32(as_h2(uu.y) * s2[mt][rt]);
            uu.z = as_u32(as_h2(uu.z) * s2[mt][rt]);
            uu.w = as_u32(as_h2(uu.w) * s2[mt][rt]);
            u = __builtin_bit_cast(h8_t, uu);
          }
          wa[mt][rt] = u;
        }
    };
    constexpr int NMF = NMAT * RT * TT;   // matrix instructions per sub-step
    auto mfma_all = [&](const h8_t (&wa)[NMAT][RT], const h8_t* xb) {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            acc[mt][rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[mt][rt], xb[tt], acc[mt][rt][tt], 0, 0, 0);
    };
    if constexpr (Q != CQ_QUANT_FP16) {
      // Software pipeline over the four sub-steps: the B fragments (LDS) and
      // A fragments (unpack) of sub-step s4 + 1 are produced while the
      // matrix instructions of s4 run; the scheduling groups interleave them
      // (the LDS reads first, then one matrix instruction and two vector
      // instructions at a time) so the unpack co-executes with the matrix
      // cores instead of alternating with them.  (The fp16 weight registers
      // leave no room for the second fragment set.)
      h8_t xb[2][TT];
      h8_t wa[2][NMAT][RT];
      read_b(0, xb[0]);
      unpack_a(0, wa[0]);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        __builtin_amdgcn_sched_barrier(0);
        if (s4 < 3) {
          read_b(s4 + 1, xb[(s4 + 1) & 1]);
          unpack_a(s4 + 1, wa[(s4 + 1) & 1]);
        }
        mfma_all(wa[s4 & 1], xb[s4 & 1]);
        if (s4 < 3) {
          __builtin_amdgcn_sched_group_barrier(0x100, TT, 0);   // LDS reads
#pragma unroll
          for (int i = 0; i < NMF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one matrix instruction
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two vector instructions
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        h8_t xb[TT];
        h8_t wa[NMAT][RT];
        read_b(s4, xb);
        unpack_a(s4, wa);
        mfma_all(wa, xb);
      }
    }
  };
  int ks = kb;
  for (; ks + 1 < ke; ks += 2) {
    step(std::integral_constant<int, 0>{}, ks);
    step(std::integral_constant<int, 1>{}, ks + 1);
  }
  if (ks < ke) step(std::integral_constant<int, 0>{}, ks);
  __syncthreads();   // every wave's last LDS reads are done before the QKV epilogue reuses the buffers

  if constexpr (SPLIT) {
    // fp32 partial [z][mat][M][N]; the split epilogue sums and finishes
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          const int n = nw0 + rt * 16 + 4 * j, m = m0 + tt * 16 + r;
          if (m < a.M && n + 3 < a.N) {
            *reinterpret_cast<f4_t*>(&a.part[(((int64_t)blockIdx.z * NMAT + mt) * a.M + m) * a.N + n]) = acc[mt][rt][tt];
          } else if (m < a.M) {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (n + v < a.N) a.part[(((int64_t)blockIdx.z * NMAT + mt) * a.M + m) * a.N + n + v] = acc[mt][rt][tt][v];
          }
        }
    return;
  }

  // ---- epilogues: lane holds rows nw0 + rt*16 + 4j + v, token m0 + tt*16 + r.
  // The residual and SwiGLU outputs go through LDS (the activation buffers,
  // free after the loop's last barrier) so that every token row is read and
  // written in 16-byte pieces rather than 2 bytes per lane.
  if constexpr (MODE == GM_RESID) {
    // fp32 sums, 64 tokens per pass: x = half(x + y), residual stays fp16 (kernels.cu:621)
    constexpr int LDF = BN + 4;   // padded fp32 row
    constexpr int HT = kPfTok / 2;
    static_assert(HT * LDF * 2 <= SM, "residual staging fits");
    float* ft = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h) __syncthreads();
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tt = h * TT / 2; tt < (h + 1) * TT / 2; ++tt)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            ft[(tt * 16 + r - h * HT) * LDF + wave * WROWS + rt * 16 + 4 * j + v] = acc[0][rt][tt][v];
      __syncthreads();
      for (int idx = threadIdx.x; idx < HT * (BN / 4); idx += kPfThreads) {
        const int ml = idx / (BN / 4), c = idx % (BN / 4);
        const int m = m0 + h * HT + ml, n = nb0 + 4 * c;
        if (m >= a.M || n >= a.N) continue;
        _Float16* p = a.out + (int64_t)m * a.N + n;
        h4_t x = *reinterpret_cast<const h4_t*>(p);
        const f4_t y = *reinterpret_cast<const f4_t*>(&ft[ml * LDF + 4 * c]);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = (_Float16)((float)x[e] + y[e]);
        *reinterpret_cast<h4_t*>(p) = x;
      }
    }
  } else if constexpr (MODE == GM_SWIGLU) {
    constexpr int LD = BN + 8;   // padded fp16 row
    static_assert(kPfTok * LD <= SM, "swiglu staging fits");
    _Float16* ot = smem;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int nl = wave * WROWS + rt * 16 + 4 * j + v, ml = tt * 16 + r;
          const int m = min(m0 + ml, a.M - 1);
          const float s = a.inv[m];
          const float g = acc[0][rt][tt][v] * s, u = acc[1][rt][tt][v] * s;
          const float sig = 1.f / (1.f + expf(-g));   // kernels.cu:566
          // nb0 is a multiple of 8, so the layout's permutation stays inside the tile
          ot[ml * LD + pf_pos(nl, Q == CQ_QUANT_INT4)] = pf_val((float)(_Float16)((g * sig) * u), nl, Q == CQ_QUANT_INT4);
        }
    __syncthreads();
    for (int idx = threadIdx.x; idx < kPfTok * (BN / 8); idx += kPfThreads) {
      const int ml = idx / (BN / 8), c = idx % (BN / 8);
      const int m = m0 + ml, n = nb0 + 8 * c;
      if (m < a.M && n < a.N)
        *reinterpret_cast<u4_t*>(a.out + (int64_t)m * a.N + n) = *reinterpret_cast<const u4_t*>(&ot[ml * LD + 8 * c]);
    }
  } else {
    // QKV: norm scale, bias, fp16 into LDS (over the activation buffers, all
    // reads of which finished at the loop's last barrier), 64 tokens per
    // pass, token-major rows; then pairs (i, i + hd/2) of each head rotate
    // (q, k) and go to Q or the KV cache, consecutive threads taking
    // consecutive pairs of one token (so Q's stores are contiguous)
    constexpr int HT = kPfTok / 2;
    constexpr int LDQ = BN + 2;   // odd dword stride: the token-per-lane reads below are conflict-free
    static_assert(HT * LDQ <= SM, "QKV staging fits");
    _Float16* ot = smem;
    const int hd = a.head_dim, half = hd / 2;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h) __syncthreads();
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tt = h * TT / 2; tt < (h + 1) * TT / 2; ++tt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int nl = wave * WROWS + rt * 16 + 4 * j + v, ml = tt * 16 + r;
            const int n = nb0 + nl, m = min(m0 + ml, a.M - 1);
            int local;
            const int mat = pf_mat(a, min(n, a.N - 1), &local);
            const _Float16* b = a.bias[mat];
            const float y = acc[0][rt][tt][v] * a.inv[m] + (b ? (float)b[local] : 0.f);
            ot[(ml - h * HT) * LDQ + nl] = (_Float16)y;   // q/k/v are fp16 before RoPE (kernels.cu:470)
          }
      __syncthreads();
      for (int idx = threadIdx.x; idx < (BN / 2) * HT; idx += kPfThreads) {
        const int pi = idx % (BN / 2), ml = idx / (BN / 2);   // pair pi of the block's BN/2 pairs
        const int nl0 = (pi / half) * hd + pi % half, nl1 = nl0 + half;
        const int n0 = nb0 + nl0, m = m0 + h * HT + ml;
        if (n0 >= a.N || m >= a.M) continue;
        int local;
        const int mat = pf_mat(a, n0, &local);
        float y0 = (float)ot[ml * LDQ + nl0], y1 = (float)ot[ml * LDQ + nl1];
        const int pos = a.pos0 + m, i = local % hd;
        if (mat < 2) rope_rotate(y0, y1, pos, a.inv_freq[i]);
        if (a.kcache8 && mat > 0) {
          // quantized cache: rotated values back into the tile, quantized per head below
          ot[ml * LDQ + nl0] = (_Float16)y0;
          ot[ml * LDQ + nl1] = (_Float16)y1;
        } else {
          pf_qkv_store(a, mat, local, m, (_Float16)y0, (_Float16)y1);
        }
      }
      if (a.kcache8) {
        __syncthreads();
        const int heads = BN / hd;
        for (int idx = threadIdx.x; idx < heads * HT; idx += kPfThreads) {
          const int hb = idx / HT, ml = idx % HT;
          const int n0 = nb0 + hb * hd, m = m0 + h * HT + ml;
          if (n0 >= a.N || m >= a.M) continue;
          int local;
          const int mat = pf_mat(a, n0, &local);
          if (mat == 0) continue;
          float amax = 0.f;
          for (int d = 0; d < hd; ++d) amax = fmaxf(amax, fabsf((float)ot[ml * LDQ + hb * hd + d]));
          pf_kv8_store(a, mat, local / hd, a.pos0 + m, amax, [&](int d) { return (float)ot[ml * LDQ + hb * hd + d]; });
        }
      }
    }
  }
}

// Split-K epilogue of the SwiGLU GEMM: sums the S partials of each output
// and applies the fused epilogue's arithmetic.
__global__ __launch_bounds__(256) void pf_split_swiglu(const PfGemmArgs a, int S) {
  const int64_t MN = (int64_t)a.M * a.N;
  auto sum = [&](int mt, int64_t i) {
    float v = 0.f;
    for (int z = 0; z < S; ++z) v += a.part[((int64_t)z * 2 + mt) * MN + i];
    return v;
  };
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < MN; idx += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(idx / a.N), n = (int)(idx % a.N);
    const float g = sum(0, idx) * a.inv[m], u = sum(1, idx) * a.inv[m];
    const float sig = 1.f / (1.f + expf(-g));
    a.out[(int64_t)m * a.N + pf_pos(n, a.quant == CQ_QUANT_INT4)] =
        pf_val((float)(_Float16)((g * sig) * u), n, a.quant == CQ_QUANT_INT4);
  }
}

// Split-K epilogue of a residual GEMM, one block per token row (N a
// multiple of 8): x = half(x + sum of the S partials), then, when asked, the
// RMSNorm of the new row (the next GEMM's input) in the same pass.
constexpr int kPfResidThreads = 512;   // one 8-element group per thread up to 4096-wide rows
__global__ __launch_bounds__(kPfResidThreads) void pf_split_resid(const PfGemmArgs a, int S) {
  __shared__ float red[16];
  const int m = blockIdx.x;
  const int64_t MN = (int64_t)a.M * a.N;
  _Float16* xr = a.out + (int64_t)m * a.N;
  for (int g = threadIdx.x; g < a.N / 8; g += blockDim.x) {
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int z = 0; z < S; ++z) {
      const f4_t* pz = reinterpret_cast<const f4_t*>(a.part + z * MN + (int64_t)m * a.N + 8 * g);
      const f4_t p0 = pz[0], p1 = pz[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] += p0[e];
        v[4 + e] += p1[e];
      }
    }
    h8_t x = __builtin_bit_cast(h8_t, load_u4(xr + 8 * g));
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (_Float16)((float)x[e] + v[e]);   // residual stays fp16 (kernels.cu:621)
    *reinterpret_cast<u4_t*>(xr + 8 * g) = __builtin_bit_cast(u4_t, x);
  }
  // the norm reads back the groups this thread has just written
  if (a.norm_w)
    pf_norm_row(xr, a.norm_w, a.norm_eps, a.N, a.norm_out + (int64_t)m * a.N, a.norm_inv + m,
                a.quant == CQ_QUANT_INT4, red);
}

// Split-K epilogue of the QKV GEMM, blockIdx.x = token: sums the partials,
// applies the norm scale and bias (q / k / v are fp16 before RoPE,
// kernels.cu:470), rotates q and k with the token's sines and cosines
// (computed once per block) and stores q, and k / v into the cache; block y
// takes pairs [1024 y, 1024 y + 1024), four per thread.  A quantized cache takes each (k or v,
// kv head) row through one wave of the blocks past the pairs.
constexpr int kPfQkvThreads = 256;
template <int HD>
__global__ __launch_bounds__(kPfQkvThreads) void pf_split_qkv(const PfGemmArgs a, int S) {
  constexpr int HALF = HD / 2;
  __shared__ float sn[HALF], cs[HALF];
  const int m = blockIdx.x, pos = a.pos0 + m;
  const int64_t MN = (int64_t)a.M * a.N;
  for (int i = threadIdx.x; i < HALF; i += blockDim.x) rope_sincos(pos, a.inv_freq[i], &sn[i], &cs[i]);
  __syncthreads();
  const float inv = a.inv[m];
  const float* prow = a.part + (int64_t)m * a.N;
  // fp16 value of row n (bias added, before RoPE)
  auto raw = [&](int n) {
    float v = 0.f;
#pragma unroll 4
    for (int z = 0; z < S; ++z) v += prow[z * MN + n];
    int local;
    const int mat = pf_mat(a, n, &local);
    const _Float16* b = a.bias[mat];
    return (float)(_Float16)(v * inv + (b ? (float)b[local] : 0.f));
  };
  const int np_store = (a.kcache8 ? a.rows[0] : a.N) / 2;   // quantized cache: k / v rows go per head below
  const int pair_blocks = (np_store / 4 + kPfQkvThreads - 1) / kPfQkvThreads;
  if ((int)blockIdx.y < pair_blocks) {
    // four consecutive pairs (i .. i+3, i + HALF .. i + HALF + 3) per thread
    const int p = 4 * (blockIdx.y * kPfQkvThreads + threadIdx.x);
    if (p >= np_store) return;
    const int i = p % HALF, n0 = (p / HALF) * HD + i;
    int local;
    const int mat = pf_mat(a, n0, &local);
    f4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int z = 0; z < S; ++z) {
      s0 += *reinterpret_cast<const f4_t*>(prow + z * MN + n0);
      s1 += *reinterpret_cast<const f4_t*>(prow + z * MN + n0 + HALF);
    }
    const _Float16* b = a.bias[mat];
    float y0[4], y1[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      y0[e] = (float)(_Float16)(s0[e] * inv + (b ? (float)b[local + e] : 0.f));
      y1[e] = (float)(_Float16)(s1[e] * inv + (b ? (float)b[local + HALF + e] : 0.f));
      if (mat < 2) rope_apply(y0[e], y1[e], sn[i + e], cs[i + e]);
    }
    h4_t h0, h1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h0[e] = (_Float16)y0[e];
      h1[e] = (_Float16)y1[e];
    }
    if (mat == 0) {
      *reinterpret_cast<h4_t*>(a.out + (int64_t)m * a.rows[0] + local) = h0;
      *reinterpret_cast<h4_t*>(a.out + (int64_t)m * a.rows[0] + local + HALF) = h1;
    } else if (mat == 1) {   // four consecutive elements of a K row are contiguous in the tiled cache
      const int kvh = local / HD;
      *reinterpret_cast<h4_t*>(a.kcache + kv_k_offset(kvh, pos, i, a.max_seq, HD)) = h0;
      *reinterpret_cast<h4_t*>(a.kcache + kv_k_offset(kvh, pos, i + HALF, a.max_seq, HD)) = h1;
    } else {
      const int kvh = local / HD;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a.vcache[kv_v_offset(kvh, pos, i + e, a.max_seq, HD)] = h0[e];
        a.vcache[kv_v_offset(kvh, pos, i + HALF + e, a.max_seq, HD)] = h1[e];
      }
    }
  } else {
    constexpr int E = HD / kWave;   // consecutive elements per lane
    const int lane = threadIdx.x & (kWave - 1), n_kv = a.rows[1] / HD;
    const int r = (blockIdx.y - pair_blocks) * (kPfQkvThreads / kWave) + threadIdx.x / kWave;
    if (r < 2 * n_kv) {
      const int mat = 1 + r / n_kv, kvh = r % n_kv;
      const int nb = a.rows[0] + (mat == 2 ? a.rows[1] : 0) + kvh * HD;
      float x[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int d = lane * E + e, i = d % HALF;
        float y0 = raw(nb + i), y1 = raw(nb + i + HALF);
        if (mat == 1) rope_apply(y0, y1, sn[i], cs[i]);
        x[e] = (float)(_Float16)(d < HALF ? y0 : y1);
      }
      int8_t q[E];
      const float sc = a.kv_fmt == CQ_KV_FP8 ? quant_row8_wave<HD, CQ_KV_FP8>(x, q) : quant_row8_wave<HD, CQ_KV_INT8>(x, q);
      int8_t* c = mat == 1 ? a.kcache8 : a.vcache8;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int d = lane * E + e;
        c[mat == 1 ? kv8_k_offset(kvh, pos, d, a.max_seq, HD) : kv8_v_offset(kvh, pos, d, a.max_seq, HD)] = q[e];
      }
      if (lane == 0) (mat == 1 ? a.kscale : a.vscale)[(int64_t)kvh * a.max_seq + pos] = sc;
    }
  }
}

// ------------------------------------------------------ causal attention
// Block = (16 consecutive tokens, one query head): the 16 tokens are the
// columns of S^T = K Q^T; 8 waves take every 8th 32-key tile up to the last
// token's position (double-buffered like the decode kernel), keys past a
// token's own position are masked per column, and the waves merge in LDS.
// Output rows are written in the GEMM activation layout.
template <int HD>
__device__ __forceinline__ void pf_attend_tile(KVTile<HD>& t, const h8_t* qb, int ti, int t_lane, int t_max,
                                               float scale, int j, float& m, float& l, f4_t* o) {
  constexpr int KK = HD / 32, DT = HD / 16;
  f4_t s[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    s[st] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(t.ka[st][kk], qb[kk], s[st], 0, 0, 0);
  }
  const int key0 = ti * kTileKeys + 4 * j;
  float sv[8];
  float mt = -INFINITY;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = (float)(_Float16)(s[st][i] * scale);   // kernels.cu:171
      if (key0 + st * 16 + i >= t_lane) v = -INFINITY;
      sv[st * 4 + i] = v;
      mt = fmaxf(mt, v);
    }
  mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
  mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
  const float mn = fmaxf(m, mt);
  // a column can have no valid key yet (its token precedes this tile)
  const float alpha = m == -INFINITY ? 0.f : __expf(m - mn);
  m = mn;
  l *= alpha;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
  h8_t pb;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = sv[e] == -INFINITY ? 0.f : __expf(sv[e] - mn);
    l += p;
    pb[e] = (_Float16)p;
  }
  if ((ti + 1) * kTileKeys > t_max) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = ti * kTileKeys + (e < 4 ? 4 * j + e : 16 + 4 * j + e - 4);
        if (key >= t_max) t.va[dt][e] = (_Float16)0.f;
      }
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(t.va[dt], pb, o[dt], 0, 0, 0);
}

template <int HD, int KV8>   // KV8: 0 fp16 cache, else the code format of the quantized cache
__global__ __launch_bounds__(kAttnThreads) void pf_attention_kernel(const PfAttnArgs a) {
  constexpr int KK = HD / 32, DT = HD / 16;
  const int t0 = blockIdx.x * 16, hq = blockIdx.y;
  const int g = a.n_heads / a.n_kv, kvh = hq / g;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int h = lane & 15, j = lane >> 4;   // h: token column
  const int tcol = min(t0 + h, a.M - 1);
  const int t_lane = a.pos0 + tcol + 1;                       // keys visible to this column
  const int t_max = a.pos0 + min(t0 + 16, a.M);               // keys visible to the block
  const int n_tiles = (t_max + kTileKeys - 1) / kTileKeys;
  const float scale = 1.0f / sqrtf((float)HD);
  const _Float16* kbase = a.kcache + (int64_t)kvh * a.max_seq * HD;
  const _Float16* vbase = a.vcache + (int64_t)kvh * a.max_seq * HD;
  h8_t qb[KK];
  const _Float16* q = a.q + (int64_t)tcol * a.n_heads * HD + hq * HD;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) qb[kk] = __builtin_bit_cast(h8_t, load_u4(q + kk * 32 + j * 8));
  float m = -INFINITY, l = 0.f;
  f4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  int ti = wave;
  if constexpr (KV8) {
    const int8_t* kb8 = a.kcache8 + (int64_t)kvh * a.max_seq * HD;
    const int8_t* vb8 = a.vcache8 + (int64_t)kvh * a.max_seq * HD;
    const float* ksc = a.kscale + (int64_t)kvh * a.max_seq;
    const float* vsc = a.vscale + (int64_t)kvh * a.max_seq;
    const uint32_t magic = vgpr_const(0x64646464u);
    KVTile8<HD> A, B;
    if (ti < n_tiles) load_tile8<HD>(A, kb8, vb8, ksc, vsc, ti, lane);
    for (; ti < n_tiles; ti += 2 * kAttnWaves) {
      const int t1 = ti + kAttnWaves;
      if (t1 < n_tiles) load_tile8<HD>(B, kb8, vb8, ksc, vsc, t1, lane);
      attend_tile8<HD, KV8>(A, qb, ti, t_lane, scale, j, m, l, o, magic);
      if (t1 >= n_tiles) break;
      if (t1 + kAttnWaves < n_tiles) load_tile8<HD>(A, kb8, vb8, ksc, vsc, t1 + kAttnWaves, lane);
      attend_tile8<HD, KV8>(B, qb, t1, t_lane, scale, j, m, l, o, magic);
    }
  } else {
    KVTile<HD> A, B;
    if (ti < n_tiles) load_tile<HD>(A, kbase, vbase, ti, lane);
    for (; ti < n_tiles; ti += 2 * kAttnWaves) {
      const int t1 = ti + kAttnWaves;
      if (t1 < n_tiles) load_tile<HD>(B, kbase, vbase, t1, lane);
      pf_attend_tile<HD>(A, qb, ti, t_lane, t_max, scale, j, m, l, o);
      if (t1 >= n_tiles) break;
      if (t1 + kAttnWaves < n_tiles) load_tile<HD>(A, kbase, vbase, t1 + kAttnWaves, lane);
      pf_attend_tile<HD>(B, qb, t1, t_lane, t_max, scale, j, m, l, o);
    }
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);

  __shared__ float wm[kAttnWaves][16], wl[kAttnWaves][16];
  __shared__ float wo[kAttnWaves][16][HD + 1];
  if (j == 0) { wm[wave][h] = m; wl[wave][h] = l; }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) wo[wave][h][dt * 16 + 4 * j + i] = o[dt][i];
  __syncthreads();
  const int qd = a.n_heads * HD;
  for (int idx = threadIdx.x; idx < 16 * HD; idx += kAttnThreads) {
    const int c = idx / HD, d = idx % HD;
    if (t0 + c >= a.M) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, wm[w][c]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float f = wm[w][c] == -INFINITY ? 0.f : __expf(wm[w][c] - M);
      L += wl[w][c] * f;
      O += wo[w][c][d] * f;
    }
    const int k = hq * HD + d;
    a.out[(int64_t)(t0 + c) * qd + pf_pos(k, a.int4_layout)] =
        pf_val((float)(_Float16)(O * (1.0f / (L + 1e-9f))), k, a.int4_layout);
  }
}

// Causal attention with the K / V tiles shared by the query heads of a GQA
// group (fp16 cache): block = (16 consecutive tokens, one kv head), 16 waves:
// wave w owns query head kvh * g + (w % 8) and, with its partner w ^ 8, runs
// the online softmax over every key tile up to the block's last token (even
// tiles in waves 0-7, odd tiles in waves 8-15); the two halves merge in LDS
// at the end.  The tiles stream global -> registers -> LDS (a tile's K and V
// are each one contiguous 32-key block of the tiled cache), a pair of tiles
// per stage, two stages, and every head of the group reads them from LDS:
// the cache is read once per kv head instead of once per query head.
constexpr int kPfGqaWaves = 16;
template <int HD>
__global__ __launch_bounds__(kPfGqaWaves * kWave) void pf_attention_gqa_kernel(const PfAttnArgs a) {
  constexpr int KK = HD / 32, DT = HD / 16;
  constexpr int TILE = kTileKeys * HD;               // halves of K (or V) per tile
  constexpr int STAGE = 4 * TILE;                    // two tiles, K and V
  constexpr int CHUNKS = STAGE * 2 / 1024;           // 1 KB pieces per stage
  constexpr int PER_WAVE = (CHUNKS + kPfGqaWaves - 1) / kPfGqaWaves;
  constexpr int MERGE = 8 * kWave * (2 + 4 * DT);    // floats of one half's softmax state
  constexpr int SM = 2 * STAGE > 2 * MERGE ? 2 * STAGE : 2 * MERGE;
  __shared__ __align__(16) _Float16 st[SM];
  const int t0 = blockIdx.x * 16, kvh = blockIdx.y;
  const int g = a.n_heads / a.n_kv;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int head = wave & 7, half = wave >> 3;
  const int h = lane & 15, j = lane >> 4;   // h: token column
  const int t_max = a.pos0 + min(t0 + 16, a.M);   // keys visible to the block
  const int n_tiles = (t_max + kTileKeys - 1) / kTileKeys;
  const int n_steps = (n_tiles + 1) / 2;
  const _Float16* kbase = a.kcache + (int64_t)kvh * a.max_seq * HD;
  const _Float16* vbase = a.vcache + (int64_t)kvh * a.max_seq * HD;
  // A step's tile pair goes global -> registers one step ahead, then into
  // one of two LDS stages at the start of the step that reads it.  Stage
  // layout: [tile 0: K, V][tile 1: K, V]; piece c of a stage is 1 KB (the
  // pair's second tile may be past the end).
  u4_t kv[PER_WAVE];
  auto piece = [&](int i, int step, int* tt, bool* isv, int* cc) {
    const int c = i * kPfGqaWaves + wave;
    *tt = c / (CHUNKS / 2);
    const int r = c % (CHUNKS / 2);
    *isv = r >= CHUNKS / 4;
    *cc = *isv ? r - CHUNKS / 4 : r;
    return c < CHUNKS && 2 * step + *tt < n_tiles;
  };
  auto load = [&](int step) {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      int tt, cc;
      bool isv;
      if (piece(i, step, &tt, &isv, &cc))
        kv[i] = load_u4((isv ? vbase : kbase) + (int64_t)(2 * step + tt) * TILE + cc * 512 + lane * 8);
    }
  };
  auto store = [&](int step) {
    _Float16* dst = st + (step & 1) * STAGE;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      int tt, cc;
      bool isv;
      if (piece(i, step, &tt, &isv, &cc))
        *reinterpret_cast<u4_t*>(dst + tt * 2 * TILE + (isv ? TILE : 0) + cc * 512 + lane * 8) = kv[i];
    }
  };
  const bool active = head < g;
  const int hq = kvh * g + min(head, g - 1);
  const int tcol = min(t0 + h, a.M - 1);
  const int t_lane = a.pos0 + tcol + 1;                // keys visible to this column
  h8_t qb[KK];
  const _Float16* q = a.q + (int64_t)tcol * a.n_heads * HD + hq * HD;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) qb[kk] = __builtin_bit_cast(h8_t, load_u4(q + kk * 32 + j * 8));
  load(0);
  const float scale = 1.0f / sqrtf((float)HD);
  float m = -INFINITY, l = 0.f;
  f4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < n_steps; ++sp) {
    // this step's pieces (loaded during the previous step) into LDS stage
    // sp % 2, last read at step sp - 2, which every wave finished before the
    // previous barrier; then visible to all waves
    __builtin_amdgcn_s_waitcnt(0x0F70);
    store(sp);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    lds_barrier();
    if (sp + 1 < n_steps) load(sp + 1);
    const int ti = 2 * sp + half;
    if (active && ti < n_tiles) {
      const _Float16* kt = st + (sp & 1) * STAGE + half * 2 * TILE;
      const _Float16* vt = kt + TILE;
      KVTile<HD> A;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          A.ka[s2][kk] = *reinterpret_cast<const h8_t*>(kt + s2 * 16 * HD + (kk * 64 + lane) * 8);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) A.va[dt] = *reinterpret_cast<const h8_t*>(vt + (dt * 64 + lane) * 8);
      pf_attend_tile<HD>(A, qb, ti, t_lane, t_max, scale, j, m, l, o);
    }
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  // merge the odd-tile half into the even one (over the stage buffers)
  __syncthreads();
  float* mg = reinterpret_cast<float*>(st) + head * kWave * (2 + 4 * DT);
  if (half == 1 && active) {
    mg[lane] = m;
    mg[kWave + lane] = l;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) mg[(2 + 4 * dt + i) * kWave + lane] = o[dt][i];
  }
  __syncthreads();
  // the merged rows go through LDS (over the merge area, once every wave
  // has read it) so each token's g heads are written as one contiguous run
  // of 16-byte pieces
  const bool writer = half == 0 && active;
  float ov[DT][4];
  if (writer) {
    const float m1 = mg[lane], l1 = mg[kWave + lane];
    const float M = fmaxf(m, m1);
    const float f0 = m == -INFINITY ? 0.f : __expf(m - M), f1 = m1 == -INFINITY ? 0.f : __expf(m1 - M);
    const float inv = 1.0f / (l * f0 + l1 * f1 + 1e-9f);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) ov[dt][i] = (o[dt][i] * f0 + mg[(2 + 4 * dt + i) * kWave + lane] * f1) * inv;
  }
  __syncthreads();
  const int GW = g * HD;   // output halves per token of this kv head
  // [16 tokens][GW + 8]: the 16-byte pad moves consecutive token rows to
  // different bank groups (unpadded, the row stride is a multiple of the
  // 256-byte bank row and the 16 token columns' 2-byte stores collide)
  const int OS = GW + 8;
  _Float16* ot = st;
  if (writer) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = head * HD + dt * 16 + 4 * j + i;   // head * HD is a multiple of 8: the layout stays in the tile
        ot[h * OS + pf_pos(k, a.int4_layout)] = pf_val((float)(_Float16)ov[dt][i], k, a.int4_layout);
      }
  }
  __syncthreads();
  const int qd = a.n_heads * HD;
  for (int idx = threadIdx.x; idx < 16 * (GW / 8); idx += kPfGqaWaves * kWave) {
    const int c = idx / (GW / 8), p8 = idx % (GW / 8);
    if (t0 + c < a.M)
      *reinterpret_cast<u4_t*>(a.out + (int64_t)(t0 + c) * qd + kvh * GW + 8 * p8) =
          *reinterpret_cast<const u4_t*>(ot + c * OS + 8 * p8);
  }
}

// One row of a GEMM input back to natural order (the int4 layout stores each
// 8-group as [0,4,1,5,2,6,3,7] with the odd elements / 16; the scale is a
// power of two, so the round trip is exact for odd elements of magnitude at
// least 2^-10 -- smaller ones lost low bits to the subnormal range on the way
// in).
__global__ __launch_bounds__(256) void pf_row_natural(const _Float16* src, _Float16* dst, int n, bool int4) {
  for (int k = threadIdx.x; k < n; k += blockDim.x)
    dst[k] = (_Float16)((float)src[pf_pos(k, int4)] * ((int4 && (k & 1)) ? 16.0f : 1.0f));
}

// ------------------------------------------------------------------ host
int launch_pf_norm(const __half* x, const __half* w, float eps, int M, int dim, __half* A, float* inv,
                   int quant, hipStream_t stream) {
  if (M <= 0 || dim <= 0 || dim % 8) return fail(CQ_EINVAL, "prefill norm: rows must be a multiple of 8 wide");
  hipLaunchKernelGGL(pf_norm_rows, dim3(M), dim3(256), 0, stream, (const _Float16*)x, (const _Float16*)w, eps, dim,
                     (_Float16*)A, inv, quant == CQ_QUANT_INT4);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

int launch_pf_row_natural(const __half* src, __half* dst, int n, int quant, hipStream_t stream) {
  hipLaunchKernelGGL(pf_row_natural, dim3(1), dim3(256), 0, stream, (const _Float16*)src, (_Float16*)dst, n,
                     quant == CQ_QUANT_INT4);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

int launch_pf_embed(const __half* embed, const int* tokens, int M, int dim, __half* x, hipStream_t stream) {
  hipLaunchKernelGGL(pf_embed, dim3(M), dim3(256), 0, stream, reinterpret_cast<const u4_t*>(embed), tokens,
                     reinterpret_cast<u4_t*>(x), dim / 8);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

template <int Q, int MODE>
static int launch_pf_gemm_m(const PfGemmArgs& a, hipStream_t stream) {
  const int bn = PfShape<Q, MODE>::BN;
  const int gx = ((a.N + bn - 1) / bn) * ((a.M + kPfTok - 1) / kPfTok);   // row blocks x token blocks
  const int nks = a.K / kPfK, nmat = MODE == GM_SWIGLU ? 2 : 1;
  // Split K when it shortens the GEMM plus its split epilogue.  Model: one
  // block fits a CU (its LDS), so B blocks take ceil(B / CUs) rounds and S
  // splits ceil(S B / CUs) rounds of 1/S the work; a full-K block runs at
  // ~4.2 TFLOP/s per CU (measured: int4 gate/up, 56 us per round of 256
  // blocks at K = 3584); the split epilogue reads the S fp32 partials at
  // ~2.8 TB/s after a launch of ~2 us (measured: QKV's 3 x 18.9 MB in 20.4
  // us, the residual's 2 x 14.7 MB in 10.7 us).  Within the workspace.
  int S = 1;
  if (a.part) {
    auto rounds = [&](int s) { return (double)(((int64_t)gx * s + kNumCUs - 1) / kNumCUs); };
    const double t1 = (double)bn * nmat * kPfTok * a.K * 2 / 4.2e6;     // us, one round of full-K blocks
    const double part_us = (double)nmat * a.M * a.N * sizeof(float) / 2.8e6;   // us per split of partials
    // QKV's unsplit epilogue (RoPE through an LDS tile, scattered cache
    // stores) costs about what the split epilogue's pass does (measured: at
    // 1024 tokens the unsplit QKV launch took ~25 us longer than the 3-way
    // split plus its epilogue)
    double best = rounds(1) * t1 + (MODE == GM_QKV ? part_us + 2.0 : 0.0);
    for (int s = 2; s <= std::min(kPfMaxSplit, nks); ++s) {
      if ((size_t)s * nmat * a.M * a.N * sizeof(float) > a.part_bytes) break;
      const double t = rounds(s) / s * t1 + s * part_us + 2.0;
      if (t < best) { best = t; S = s; }
    }
  }
  if (S > 1) {
    hipLaunchKernelGGL((pf_gemm_kernel<Q, MODE, true>), dim3(gx, 1, S), dim3(kPfThreads), 0, stream, a);
    CQ_HIP(hipGetLastError());
    if constexpr (MODE == GM_QKV) {
      const int np_store = (a.kcache8 ? a.rows[0] : a.N) / 2, waves = kPfQkvThreads / kWave;
      const int ny = (np_store / 4 + kPfQkvThreads - 1) / kPfQkvThreads +
                     (a.kcache8 ? (2 * (a.rows[1] / a.head_dim) + waves - 1) / waves : 0);
      if (a.head_dim == 128) hipLaunchKernelGGL((pf_split_qkv<128>), dim3(a.M, ny), dim3(kPfQkvThreads), 0, stream, a, S);
      else hipLaunchKernelGGL((pf_split_qkv<64>), dim3(a.M, ny), dim3(kPfQkvThreads), 0, stream, a, S);
    } else if constexpr (MODE == GM_RESID) {
      hipLaunchKernelGGL(pf_split_resid, dim3(a.M), dim3(kPfResidThreads), 0, stream, a, S);
    } else {
      const int eb = (int)std::min<int64_t>(((int64_t)a.M * a.N + 255) / 256, 4096);
      hipLaunchKernelGGL(pf_split_swiglu, dim3(eb), dim3(256), 0, stream, a, S);
    }
  } else {
    hipLaunchKernelGGL((pf_gemm_kernel<Q, MODE, false>), dim3(gx), dim3(kPfThreads), 0, stream, a);
    if (MODE == GM_RESID && a.norm_w) {
      CQ_HIP(hipGetLastError());
      hipLaunchKernelGGL(pf_norm_rows, dim3(a.M), dim3(256), 0, stream, (const _Float16*)a.out, a.norm_w, a.norm_eps,
                         a.N, a.norm_out, a.norm_inv, Q == CQ_QUANT_INT4);
    }
  }
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

template <int Q>
static int launch_pf_gemm_q(const PfGemmArgs& a, hipStream_t stream) {
  if (a.mode == GM_QKV) return launch_pf_gemm_m<Q, GM_QKV>(a, stream);
  if (a.mode == GM_SWIGLU) return launch_pf_gemm_m<Q, GM_SWIGLU>(a, stream);
  return launch_pf_gemm_m<Q, GM_RESID>(a, stream);
}

int launch_pf_gemm(const PfGemmArgs& a, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.K % kPfK) return fail(CQ_EINVAL, "prefill gemm: K must be a multiple of 128");
  if (!a.A || !a.W[0] || !a.out) return fail(CQ_EINVAL, "prefill gemm: null operand");
  if (a.quant != CQ_QUANT_FP16 && !a.S[0]) return fail(CQ_EINVAL, "prefill gemm: quantized weights need scales");
  if (a.mode == GM_SWIGLU && (!a.W[1] || !a.inv || a.N % 8))
    return fail(CQ_EINVAL, "prefill gemm: swiglu needs gate, up, the norm and rows a multiple of 8");
  if (a.mode == GM_RESID && (a.N % 8 || (a.norm_w && (!a.norm_out || !a.norm_inv))))
    return fail(CQ_EINVAL, "prefill gemm: residual rows must be a multiple of 8 wide; the norm needs its outputs");
  if (a.panels && a.mode != GM_RESID) return fail(CQ_EINVAL, "prefill gemm: paneled weights are a residual-mode option");
  if (a.mode == GM_QKV) {
    if (!a.inv || !a.W[1] || !a.W[2] || !a.inv_freq) return fail(CQ_EINVAL, "prefill gemm: qkv operands");
    if (a.kcache8 ? (!a.vcache8 || !a.kscale || !a.vscale) : (!a.kcache || !a.vcache))
      return fail(CQ_EINVAL, "prefill gemm: qkv cache pointers");
    if (PfShape<CQ_QUANT_FP16, GM_QKV>::BN % a.head_dim || a.rows[0] % a.head_dim || a.rows[1] % a.head_dim || a.rows[0] + a.rows[1] + a.rows[2] != a.N)
      return fail(CQ_EINVAL, "prefill gemm: qkv rows must be whole heads");
  }
  switch (a.quant) {
    case CQ_QUANT_FP16: return launch_pf_gemm_q<CQ_QUANT_FP16>(a, stream);
    case CQ_QUANT_INT8: return launch_pf_gemm_q<CQ_QUANT_INT8>(a, stream);
    default: return launch_pf_gemm_q<CQ_QUANT_INT4>(a, stream);
  }
}

int launch_pf_attention(const PfAttnArgs& a, hipStream_t stream) {
  if (a.head_dim != 64 && a.head_dim != 128) return fail(CQ_EINVAL, "prefill attention: head_dim must be 64 or 128");
  if (a.M <= 0 || a.pos0 < 0 || a.pos0 + a.M > a.max_seq) return fail(CQ_ERANGE, "prefill attention: positions");
  const dim3 grid((a.M + 15) / 16, a.n_heads);
  if (a.kcache8) {
    if (!a.vcache8 || !a.kscale || !a.vscale) return fail(CQ_EINVAL, "prefill attention: quantized cache pointers");
    if (a.kv_fmt == CQ_KV_FP8) {
      if (a.head_dim == 128) hipLaunchKernelGGL((pf_attention_kernel<128, CQ_KV_FP8>), grid, dim3(kAttnThreads), 0, stream, a);
      else hipLaunchKernelGGL((pf_attention_kernel<64, CQ_KV_FP8>), grid, dim3(kAttnThreads), 0, stream, a);
    } else {
      if (a.head_dim == 128) hipLaunchKernelGGL((pf_attention_kernel<128, CQ_KV_INT8>), grid, dim3(kAttnThreads), 0, stream, a);
      else hipLaunchKernelGGL((pf_attention_kernel<64, CQ_KV_INT8>), grid, dim3(kAttnThreads), 0, stream, a);
    }
  } else if (a.n_heads / a.n_kv <= 8) {
    const dim3 g2((a.M + 15) / 16, a.n_kv);
    if (a.head_dim == 128) hipLaunchKernelGGL((pf_attention_gqa_kernel<128>), g2, dim3(kPfGqaWaves * kWave), 0, stream, a);
    else hipLaunchKernelGGL((pf_attention_gqa_kernel<64>), g2, dim3(kPfGqaWaves * kWave), 0, stream, a);
  } else {
    if (a.head_dim == 128) hipLaunchKernelGGL((pf_attention_kernel<128, 0>), grid, dim3(kAttnThreads), 0, stream, a);
    else hipLaunchKernelGGL((pf_attention_kernel<64, 0>), grid, dim3(kAttnThreads), 0, stream, a);
  }
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

}  // namespace cq
