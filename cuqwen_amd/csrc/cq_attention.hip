// FlashDecoding GQA attention over the fp16 KV cache for gfx950.
//
// Reference: gqa_attention_wmma_ksplit_stage1_kernel + stage2
// (src/kernels.cu:105-324).  Design here:
//   * stage 1: grid = (partitions, kv heads); a partition is a run of 32-key
//     tiles, sized at run time from *d_pos so one recorded graph serves every
//     position; blocks past the last partition exit at once;
//   * 8 waves per block, each wave takes every 8th tile of the partition,
//     double-buffered in registers (the next tile's K and V are in flight
//     while the current one is computed), and keeps an online softmax
//     (running max / sum) and its O accumulator in matrix-core registers;
//   * S^T = K Q^T with v_mfma_f32_16x16x32_f16 (keys as rows, the group's
//     query heads as columns, padded to 16), then O^T += V^T P^T with the
//     same instruction.  The K and V tiles are stored in the cache in exactly
//     the operand order the instruction consumes (cq_common.h), so every
//     tile is streamed with contiguous 16-byte-per-lane loads and the score
//     tile feeds the P^T operand without any cross-lane movement;
//   * the 8 waves merge in LDS and the block writes one (m, l, O) partial
//     (or, with a single partition, the output itself);
//   * stage 2: one wave per (query head, 16-dim slice) merges the partials
//     with the log-sum-exp rule (kernels.cu:222-288).  A separate launch is cheaper on
//     this part than an in-kernel completion ticket plus device-scope fences.
// Rounding follows the reference: scores are rounded to fp16 after the
// 1/sqrt(hd) scale (kernels.cu:171), probabilities are rounded to fp16 for
// the PV product while the row sum uses the unrounded values (:185-186).
#include "cq_attention.h"

#include <cmath>

namespace cq {

int attention_max_parts(int n_kv) { return (kAttnBlocksTarget + n_kv - 1) / n_kv; }

// Workspace: [m: n_kv*16*P] [l: n_kv*16*P] [o: n_kv*16*P*hd] floats, slot
// (kv head * 16 + head within the group) * P + partition.
size_t attention_workspace_bytes(int n_heads, int n_kv, int head_dim) {
  (void)n_heads;
  const size_t P = (size_t)attention_max_parts(n_kv);
  return (size_t)n_kv * P * 16 * (2 + (size_t)head_dim) * sizeof(float);
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attention_stage1(const AttnArgs a) {
  pin_attn_args<false>(a);
  constexpr int KK = HD / 32;
  constexpr int DT = HD / 16;
  const int kvh = blockIdx.y;
  const int part = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform, so the tile loop is a scalar loop with exact load counts
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = a.n_heads / a.n_kv;
  const int T = (int)load_ctl_u32(a.d_pos) + 1;
  const int n_tiles = (T + kTileKeys - 1) / kTileKeys;
  int tpp;
  const int nparts = attn_nparts(T, gridDim.x, &tpp);
  if (part >= nparts) return;
  const int tile0 = part * tpp;
  const int tile1 = min(tile0 + tpp, n_tiles);

  const int h = lane & 15;        // query head column of this lane
  const int j = lane >> 4;        // k-slot group of this lane

  const _Float16* kbase = reinterpret_cast<const _Float16*>(a.kcache) + (int64_t)kvh * a.max_seq * HD;
  const _Float16* vbase = reinterpret_cast<const _Float16*>(a.vcache) + (int64_t)kvh * a.max_seq * HD;

  const KVRes kv{kbase, vbase, a.max_seq * HD * 2};
  KVTile<HD> A, B;
  int ti = tile0 + wave;
  load_tile<HD>(A, kv, ti, ti < tile1, lane);

  // Q^T as the B operand: lane holds q[h][kk*32 + j*8 .. +8]
  h8_t qb[KK];
  {
    const _Float16* q = reinterpret_cast<const _Float16*>(a.q) + (int64_t)(kvh * g + h) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (h < g) qb[kk] = __builtin_bit_cast(h8_t, load_u4(q + kk * 32 + j * 8));
      else qb[kk] = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  float m = -INFINITY, l = 0.f;
  f4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  attend_partition<HD>(A, B, qb, ti, tile1, T, kv, lane, m, l, o);
  block_merge_write<HD>(a, kvh, part, nparts, g, m, l, o);
}

// Stage 1 over a quantized cache (format F: int8 or E4M3 codes).  The wave whose tiles include the step's new
// position quantizes the new k / v rows of its kv head (one row per
// wave reduction), writes them and their scales into the cache for later
// steps, and patches them into its loaded tile: no other wave of the launch
// reads that position, so no block synchronisation is needed.
template <int HD, int F>
__global__ __launch_bounds__(kAttnThreads) void attention_stage1_kv8(const AttnArgs a) {
  pin_attn_args<true>(a);
  constexpr int KK = HD / 32, DT = HD / 16, E = HD / kWave;
  const int kvh = blockIdx.y, part = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);   // scalar tile loop
  const int g = a.n_heads / a.n_kv;
  const int pos = (int)load_ctl_u32(a.d_pos), T = pos + 1;
  const int n_tiles = (T + kTileKeys - 1) / kTileKeys;
  int tpp;
  const int nparts = attn_nparts(T, gridDim.x, &tpp);
  if (part >= nparts) return;
  const int tile0 = part * tpp, tile1 = min(tile0 + tpp, n_tiles);
  const int h = lane & 15, j = lane >> 4;
  const float scale = 1.0f / sqrtf((float)HD);
  const uint32_t magic = vgpr_const(0x64646464u);
  const int8_t* kbase = a.kcache8 + (int64_t)kvh * a.max_seq * HD;
  const int8_t* vbase = a.vcache8 + (int64_t)kvh * a.max_seq * HD;
  const float* ksc = a.kscale + (int64_t)kvh * a.max_seq;
  const float* vsc = a.vscale + (int64_t)kvh * a.max_seq;

  // The new row (position pos) belongs to tile n_tiles - 1 of the last
  // partition.  Its owner wave requests the fp16 k / v rows before anything
  // else: loads complete in issue order for the wave, so issued after the
  // tiles they would wait for the whole tile prefetch, and the quantization
  // below would then sit on the kernel's critical path instead of running
  // while the tiles are in flight.
  const int last = n_tiles - 1;
  const bool owns_new = part == nparts - 1 && ((last - tile0) % kAttnWaves) == wave;
  float xnew[2][E];
  if (owns_new) {
#pragma unroll
    for (int kind = 0; kind < 2; ++kind) {
      const _Float16* src = reinterpret_cast<const _Float16*>(kind ? a.v_new : a.k_new) + (int64_t)kvh * HD + lane * E;
#pragma unroll
      for (int i = 0; i < E; ++i) xnew[kind][i] = (float)src[i];
    }
  }
  // codes and scales through buffer resources (KVRes8): the loop issues the
  // same loads on every path, so each wait names only the tile attended
  const KVRes8 kv{kbase, vbase, ksc, vsc, a.max_seq * HD, a.max_seq * 4};
  KVTile8<HD> A, B;
  int ti = tile0 + wave;
  load_tile8<HD>(A, kv, ti, ti < tile1, lane);
  h8_t qb[KK];
  {
    const _Float16* q = reinterpret_cast<const _Float16*>(a.q) + (int64_t)(kvh * g + h) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (h < g) qb[kk] = __builtin_bit_cast(h8_t, load_u4(q + kk * 32 + j * 8));
      else qb[kk] = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  // The owner quantizes the new rows while its first tile is in flight and
  // patches them into its loaded tile (the tile's copy of that position is
  // replaced, so whether the load saw the old or the new bytes does not
  // matter); the codes and scales also go to the cache for later steps.
  __shared__ __align__(16) int8_t newq[2][HD];
  __shared__ float news[2];
  if (owns_new) {
#pragma unroll
    for (int kind = 0; kind < 2; ++kind) {
      int8_t qv[E];
      const float sc = quant_row8_wave<HD, F>(xnew[kind], qv);
      int8_t* cache = kind ? a.vcache8 : a.kcache8;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int d = lane * E + i;
        newq[kind][d] = qv[i];
        cache[kind ? kv8_v_offset(kvh, pos, d, a.max_seq, HD) : kv8_k_offset(kvh, pos, d, a.max_seq, HD)] = qv[i];
      }
      if (lane == 0) {
        news[kind] = sc;
        (kind ? a.vscale : a.kscale)[(int64_t)kvh * a.max_seq + pos] = sc;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  float m = -INFINITY, l = 0.f;
  f4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  const int kp = pos & (kTileKeys - 1);
  for (; ti < tile1; ti += 2 * kAttnWaves) {
    const int t1 = ti + kAttnWaves;
    load_tile8<HD>(B, kv, t1, t1 < tile1, lane);
    if (owns_new && ti == last) patch_key8<HD>(A, kp, newq[0], newq[1], news[0], news[1], lane);
    attend_tile8<HD, F>(A, qb, ti, T, scale, j, m, l, o, magic);
    if (t1 >= tile1) break;
    load_tile8<HD>(A, kv, t1 + kAttnWaves, t1 + kAttnWaves < tile1, lane);
    if (owns_new && t1 == last) patch_key8<HD>(B, kp, newq[0], newq[1], news[0], news[1], lane);
    attend_tile8<HD, F>(B, qb, t1, T, scale, j, m, l, o, magic);
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  block_merge_write<HD>(a, kvh, part, nparts, g, m, l, o);
}

// Stage 2: log-sum-exp merge of the partitions (kernels.cu:222-288) with
// 1/(L + 1e-9).  One wave per (query head, 16-dim slice), so the few MB of
// partials are spread over n_heads * hd/16 CUs instead of n_heads; lane p
// holds partition p (64 partitions per round, merged into a running
// (M, L, O) when there are more), and every load of a round is issued
// before any is used.  The sums are DPP wave reductions.
constexpr int kMergeDims = 16;
template <int HD>
__global__ __launch_bounds__(kWave) void attention_stage2(const AttnArgs a, int Pmax) {
  constexpr int NS = HD / kMergeDims;
  const int hq = blockIdx.x / NS, d0 = (blockIdx.x % NS) * kMergeDims;
  const int g = a.n_heads / a.n_kv;
  const int kvh = hq / g, hh = hq % g;
  const int lane = threadIdx.x;
  const float* ws_m = reinterpret_cast<const float*>(a.workspace);
  const float* ws_l = ws_m + (size_t)a.n_kv * Pmax * 16;
  const float* ws_o = ws_l + (size_t)a.n_kv * Pmax * 16;
  const size_t base = ((size_t)kvh * 16 + hh) * Pmax;   // head-major slots
  // the first round's slots (partition = lane) are requested before the
  // position is known: they do not depend on it, and slots past the
  // partition count are masked below (selected out, so stale contents of
  // unused slots never reach the sums)
  auto load_round = [&](int p0, float& mp, float& lp, f4_t* ov) {
    const size_t slot = base + min(p0 + lane, Pmax - 1);
    mp = ws_m[slot];
    lp = ws_l[slot];
    const f4_t* op = reinterpret_cast<const f4_t*>(ws_o + slot * HD + d0);
#pragma unroll
    for (int i = 0; i < kMergeDims / 4; ++i) ov[i] = op[i];
  };
  float mp, lp;
  f4_t ov[kMergeDims / 4];
  load_round(0, mp, lp, ov);
  const int T = (int)load_ctl_u32(a.d_pos) + 1;
  int tpp;
  const int nparts = attn_nparts(T, Pmax, &tpp);
  if (nparts == 1) return;   // stage 1 wrote the output
  float M = -INFINITY, L = 0.f, O[kMergeDims];
#pragma unroll
  for (int i = 0; i < kMergeDims; ++i) O[i] = 0.f;
  for (int p0 = 0; p0 < nparts; p0 += kWave) {
    if (p0 > 0) load_round(p0, mp, lp, ov);
    const bool valid = p0 + lane < nparts && mp != -INFINITY;
    const float Mn = fmaxf(M, wave_max(valid ? mp : -INFINITY));
    const float f = M == -INFINITY ? 0.f : __expf(M - Mn);
    const float w = valid ? __expf(mp - Mn) : 0.f;
    L = L * f + wave_sum(valid ? lp * w : 0.f);
#pragma unroll
    for (int i = 0; i < kMergeDims / 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) O[4 * i + e] = O[4 * i + e] * f + wave_sum(valid ? ov[i][e] * w : 0.f);
    M = Mn;
  }
  const float inv = 1.0f / (L + 1e-9f);
  _Float16* out = reinterpret_cast<_Float16*>(a.out) + (int64_t)hq * HD + d0;
#pragma unroll
  for (int i = 0; i < kMergeDims; ++i)
    if (lane == i) out[i] = (_Float16)(O[i] * inv);
}

static int attention_check(const AttnArgs& a) {
  if (a.head_dim != 64 && a.head_dim != 128) return fail(CQ_EINVAL, "attention: head_dim must be 64 or 128");
  if (a.n_kv <= 0 || a.n_heads % a.n_kv || a.n_heads / a.n_kv > 16 || a.n_kv > 64)
    return fail(CQ_EINVAL, "attention: need n_heads/n_kv_heads <= 16 and n_kv_heads <= 64");
  if (a.max_seq <= 0 || a.max_seq % kTileKeys) return fail(CQ_EINVAL, "attention: max_seq_len must be a multiple of 32");
  // one kv head's K (or V) slice is read as a buffer resource (32-bit size)
  if ((int64_t)a.max_seq * a.head_dim * 2 >= ((int64_t)1 << 31)) return fail(CQ_EINVAL, "attention: max_seq_len too large");
  const bool kv8 = a.kcache8 != nullptr;
  if (!a.q || !a.out || !a.d_pos || !a.workspace) return fail(CQ_EINVAL, "attention: null pointer");
  if (kv8 && a.kv_fmt != CQ_KV_INT8 && a.kv_fmt != CQ_KV_FP8) return fail(CQ_EINVAL, "attention: unknown KV code format");
  if (kv8 ? (!a.vcache8 || !a.kscale || !a.vscale || !a.k_new || !a.v_new) : (!a.kcache || !a.vcache))
    return fail(CQ_EINVAL, "attention: null cache pointer");
  return CQ_OK;
}

int launch_attention_stage1(const AttnArgs& a, hipStream_t stream) {
  CQ_TRY(attention_check(a));
  const bool kv8 = a.kcache8 != nullptr;
  const int P = attention_max_parts(a.n_kv);
  const dim3 grid(P, a.n_kv);
  if (kv8 && a.kv_fmt == CQ_KV_FP8) {
    if (a.head_dim == 128) hipLaunchKernelGGL((attention_stage1_kv8<128, CQ_KV_FP8>), grid, dim3(kAttnThreads), 0, stream, a);
    else hipLaunchKernelGGL((attention_stage1_kv8<64, CQ_KV_FP8>), grid, dim3(kAttnThreads), 0, stream, a);
  } else if (kv8) {
    if (a.head_dim == 128) hipLaunchKernelGGL((attention_stage1_kv8<128, CQ_KV_INT8>), grid, dim3(kAttnThreads), 0, stream, a);
    else hipLaunchKernelGGL((attention_stage1_kv8<64, CQ_KV_INT8>), grid, dim3(kAttnThreads), 0, stream, a);
  } else {
    if (a.head_dim == 128) hipLaunchKernelGGL(attention_stage1<128>, grid, dim3(kAttnThreads), 0, stream, a);
    else hipLaunchKernelGGL(attention_stage1<64>, grid, dim3(kAttnThreads), 0, stream, a);
  }
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

int launch_attention(const AttnArgs& a, hipStream_t stream) {
  CQ_TRY(launch_attention_stage1(a, stream));
  const int P = attention_max_parts(a.n_kv);
  if (a.head_dim == 128)
    hipLaunchKernelGGL(attention_stage2<128>, dim3(a.n_heads * (128 / kMergeDims)), dim3(kWave), 0, stream, a, P);
  else
    hipLaunchKernelGGL(attention_stage2<64>, dim3(a.n_heads * (64 / kMergeDims)), dim3(kWave), 0, stream, a, P);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

}  // namespace cq
