// Decode attention and KV store over the reference's head-major cache
// [n_kv][max_seq][head_dim] fp16 (src/model.cu:112-114), for callers that keep
// the reference's layout and its partial buffers at the op level
// (launch_gqa_attention_decode / launch_kv_cache_store,
// include/kernels.cuh:21-47).  The engine's own step uses the MFMA-tiled
// cache of cq_attention.hip; this path exists so that a head-major cache is
// read correctly instead of being misread as tiled.
//
// Stage 1: grid (n_kv, 64 partitions) like kernels.cu:290-324, partition p
// covering keys [p*chunk, min((p+1)*chunk, T)) with chunk = ceil(T/64), on
// the matrix cores (attention_hm_mfma_stage1 below); the block writes the
// partition's (max, sum, unnormalised O) at the reference's partial index
// (kv_head * 16 + head) * 64 + partition (kernels.cuh:10-16).
// Stage 2: one wave per (query head, 16 dims), lane = partition, log-sum-exp
// merge with 1 / (L + 1e-9) (kernels.cu:222-288).
#include "cq_attention.h"
#include "cq_device.h"
#include "cq_internal.h"

namespace cq {

constexpr int kHmParts = 64;      // ATTN_PARTITIONS (include/config.h:146)
constexpr int kHmSlots = 16;      // PARTIAL_HEAD_SLOTS (include/kernels.cuh:16)

// Orders this wave's LDS writes before its later LDS reads (lanes read what
// other lanes of the same wave wrote).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Stage 1 on the matrix cores over the head-major cache, with the
// reference's partitions (64 per kv head, chunk = ceil(T/64) keys from
// p * chunk) and partial buffers.  The engine's tiled kernel does the same
// work over its MFMA-ordered cache; here the operands are formed from the
// reference's row-per-key layout:
//   * K: the A operand of S^T = K Q^T takes 8 consecutive dims of one key
//     per lane, which is 16 contiguous bytes of a head-major K row, so K
//     tiles are loaded straight into operand registers;
//   * V: the A operand of O^T += V^T P^T needs 8 keys of one dim per lane,
//     which the head-major layout strides 2*head_dim bytes apart.  V rows
//     are loaded coalesced (16 bytes per lane), stored in a per-wave LDS
//     tile whose row is the key's slot in the order the score accumulators
//     hand keys to each lane, and each operand is gathered from it per dim.
// Eight waves per block each take every 8th 32-key tile of the partition,
// two tiles in flight; keys past the partition are read from its last row
// and masked.  The waves merge in LDS (block_merge_store) into the
// reference's partial slots (kv_head * 16 + head) * 64 + partition.
template <int HD>
struct HmTile {
  u4_t k[2][HD / 32];               // K operand pieces: 16 keys x 8 dims per lane, two 16-key halves
  u4_t v[32 * HD / (kWave * 8)];    // V rows: 8 dims of one key per lane and load
};

template <int HD>
__device__ __forceinline__ void hm_load_tile(HmTile<HD>& t, const _Float16* kbase, const _Float16* vbase, int k0,
                                             int last, int lane) {
  constexpr int LPK = HD / 8, KPI = kWave / LPK;   // lanes per V row, V rows per load
  const int r = lane & 15, j = lane >> 4;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int key = min(k0 + st * 16 + r, last);
#pragma unroll
    for (int kk = 0; kk < HD / 32; ++kk) t.k[st][kk] = load_u4_stream(kbase + (int64_t)key * HD + kk * 32 + j * 8);
  }
#pragma unroll
  for (int i = 0; i < 32 / KPI; ++i) {
    const int key = min(k0 + i * KPI + lane / LPK, last);
    t.v[i] = load_u4_stream(vbase + (int64_t)key * HD + (lane % LPK) * 8);
  }
}

// slot of key k (0..31) in a lane's 8-key P^T / V^T operand order: lane
// group j holds keys 4j..4j+3 and 16+4j..16+4j+3
__device__ __forceinline__ int hm_slot(int k) { return ((k & 15) >> 2) * 8 + (k & 3) + ((k >> 4) << 2); }

template <int HD>
__device__ __forceinline__ void hm_attend_tile(HmTile<HD>& t, _Float16* vt, const h8_t* qb, int k0, int t_end,
                                               float scale, int lane, float& m, float& l, f4_t* o) {
  constexpr int KK = HD / 32, DT = HD / 16, VS = HD + 8;   // V tile row in LDS: one key slot, padded
  constexpr int LPK = HD / 8, KPI = kWave / LPK;
  const int j = lane >> 4;
  f4_t s[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    s[st] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, t.k[st][kk]), qb[kk], s[st], 0, 0, 0);
  }
  // lane holds S^T[key = k0 + st*16 + 4j + i][head]; the reference rounds the
  // scaled score to fp16 (kernels.cu:171)
  float sv[8];
  float mt = -INFINITY;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = (float)(_Float16)(s[st][i] * scale);
      if (k0 + st * 16 + 4 * j + i >= t_end) v = -INFINITY;
      sv[st * 4 + i] = v;
      mt = fmaxf(mt, v);
    }
  mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
  mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
  const float mn = fmaxf(m, mt);   // finite: key k0 is always in the partition
  const float alpha = __expf(m - mn);
  m = mn;
  l *= alpha;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
  h8_t pb;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = __expf(sv[e] - mn);
    l += p;
    pb[e] = (_Float16)p;   // P in fp16 for the PV product, the sum unrounded (kernels.cu:185-186)
  }
  // V rows -> LDS as whole 16-byte pieces, row = the key's operand slot
  // (after the scores: the V loads were issued after the K loads, so the
  // scores need not wait for them); the operands are then gathered per dim.
  // The padded row (HD + 8 halves) puts the four slot groups j of a read on
  // different banks.
#pragma unroll
  for (int i = 0; i < 32 / KPI; ++i) {
    const int d0 = (lane % LPK) * 8, slot = hm_slot(i * KPI + lane / LPK);
    *reinterpret_cast<u4_t*>(vt + slot * VS + d0) = t.v[i];
  }
  wave_lds_sync();
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    h8_t va;
#pragma unroll
    for (int e = 0; e < 8; ++e) va[e] = vt[(j * 8 + e) * VS + dt * 16 + (lane & 15)];
    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[dt], 0, 0, 0);
  }
  wave_lds_sync();   // the next tile rewrites vt
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attention_hm_mfma_stage1(
    const __half* __restrict__ q, const __half* __restrict__ kc, const __half* __restrict__ vc,
    float* __restrict__ part_out, float* __restrict__ part_max, float* __restrict__ part_sum,
    const int* __restrict__ d_pos, int n_heads, int n_kv, int max_seq) {
  constexpr int KK = HD / 32, DT = HD / 16, VS = HD + 8;
  const int kvh = blockIdx.x, part = blockIdx.y;
  const int g = n_heads / n_kv;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int T = (int)load_ctl_u32(d_pos) + 1;
  const int chunk = (T + kHmParts - 1) / kHmParts;
  const int t0 = part * chunk, t1 = min(t0 + chunk, T);
  if (t0 >= t1) return;   // block-uniform: no barrier has been reached yet
  const int n_tiles = (t1 - t0 + kTileKeys - 1) / kTileKeys;
  const int h = lane & 15, j = lane >> 4;
  const _Float16* kbase = reinterpret_cast<const _Float16*>(kc) + (int64_t)kvh * max_seq * HD;
  const _Float16* vbase = reinterpret_cast<const _Float16*>(vc) + (int64_t)kvh * max_seq * HD;
  __shared__ __align__(16) _Float16 vts[kAttnWaves][kTileKeys * VS];
  _Float16* vt = vts[wave];

  HmTile<HD> A, B;
  int ti = wave;
  if (ti < n_tiles) hm_load_tile<HD>(A, kbase, vbase, t0 + ti * kTileKeys, t1 - 1, lane);
  h8_t qb[KK];
  {
    const _Float16* qh = reinterpret_cast<const _Float16*>(q) + (int64_t)(kvh * g + h) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (h < g) qb[kk] = __builtin_bit_cast(h8_t, load_u4(qh + kk * 32 + j * 8));
      else qb[kk] = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  const float scale = 1.0f / sqrtf((float)HD);
  float m = -INFINITY, l = 0.f;
  f4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  for (; ti < n_tiles; ti += 2 * kAttnWaves) {
    const int t1i = ti + kAttnWaves;
    if (t1i < n_tiles) hm_load_tile<HD>(B, kbase, vbase, t0 + t1i * kTileKeys, t1 - 1, lane);
    hm_attend_tile<HD>(A, vt, qb, t0 + ti * kTileKeys, t1, scale, lane, m, l, o);
    if (t1i >= n_tiles) break;
    if (t1i + kAttnWaves < n_tiles) hm_load_tile<HD>(A, kbase, vbase, t0 + (t1i + kAttnWaves) * kTileKeys, t1 - 1, lane);
    hm_attend_tile<HD>(B, vt, qb, t0 + t1i * kTileKeys, t1, scale, lane, m, l, o);
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  block_merge_store<HD>(kvh, part, g, m, l, o, part_max, part_sum, part_out, kHmParts, nullptr);
}

// Stage 2: one wave per (query head, 16-dim slice), lane p holding
// partition p (the reference's 64), every load issued before any is used,
// log-sum-exp merge with DPP wave reductions and 1 / (L + 1e-9)
// (kernels.cu:222-288).
constexpr int kHmMergeDims = 16;
template <int HD>
__global__ __launch_bounds__(kWave) void attention_hm_stage2(const float* __restrict__ part_out,
                                                            const float* __restrict__ part_max,
                                                            const float* __restrict__ part_sum, __half* __restrict__ out,
                                                            const int* __restrict__ d_pos, int n_heads, int n_kv) {
  static_assert(kHmParts == kWave, "one partition per lane");
  constexpr int NS = HD / kHmMergeDims;
  const int hq = blockIdx.x / NS, d0 = (blockIdx.x % NS) * kHmMergeDims;
  const int g = n_heads / n_kv;
  const int lane = threadIdx.x;
  const size_t slot = ((size_t)(hq / g) * kHmSlots + hq % g) * kHmParts + lane;
  const float mp = part_max[slot], lp = part_sum[slot];
  f4_t ov[kHmMergeDims / 4];
#pragma unroll
  for (int i = 0; i < kHmMergeDims / 4; ++i) ov[i] = reinterpret_cast<const f4_t*>(part_out + slot * HD + d0)[i];
  const int T = (int)load_ctl_u32(d_pos) + 1;
  const int chunk = (T + kHmParts - 1) / kHmParts;
  const int nonempty = (T + chunk - 1) / chunk;
  const bool valid = lane < nonempty;   // stale slots of empty partitions never reach the sums
  const float M = wave_max(valid ? mp : -INFINITY);
  const float w = valid ? __expf(mp - M) : 0.f;
  const float L = wave_sum(valid ? lp * w : 0.f);
  const float inv = 1.0f / (L + 1e-9f);
  _Float16* o = reinterpret_cast<_Float16*>(out) + (int64_t)hq * HD + d0;
#pragma unroll
  for (int i = 0; i < kHmMergeDims / 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = wave_sum(valid ? ov[i][e] * w : 0.f);
      if (lane == 4 * i + e) o[4 * i + e] = (_Float16)(v * inv);
    }
}

__global__ void kv_store_hm_kernel(const __half* __restrict__ k, const __half* __restrict__ v, __half* __restrict__ kc,
                                   __half* __restrict__ vc, const int* __restrict__ d_pos, int n_kv, int max_seq,
                                   int hd) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_kv * hd) return;
  const int h = i / hd, d = i % hd;
  const size_t dst = ((size_t)h * max_seq + *d_pos) * hd + d;
  kc[dst] = k[i];
  vc[dst] = v[i];
}

size_t attention_hm_partial_floats(int n_kv, int head_dim) {
  return (size_t)n_kv * kHmSlots * kHmParts * (size_t)head_dim;
}

int launch_attention_hm(const __half* q, const __half* kc, const __half* vc, __half* out, const int* d_pos,
                        int n_heads, int n_kv, int head_dim, int max_seq, float* part_out, float* part_max,
                        float* part_sum, hipStream_t stream) {
  if (!q || !kc || !vc || !out || !d_pos || !part_out || !part_max || !part_sum)
    return fail(CQ_EINVAL, "attention (head-major): null pointer");
  if (head_dim != 64 && head_dim != 128) return fail(CQ_EINVAL, "attention (head-major): head_dim must be 64 or 128");
  if (n_kv <= 0 || n_heads % n_kv || n_heads / n_kv > kHmSlots)
    return fail(CQ_EINVAL, "attention (head-major): need n_heads / n_kv_heads <= 16");
  if (max_seq <= 0) return fail(CQ_EINVAL, "attention (head-major): bad max_seq_len");
  const dim3 grid(n_kv, kHmParts), block(kAttnThreads);
  if (head_dim == 128) {
    hipLaunchKernelGGL(attention_hm_mfma_stage1<128>, grid, block, 0, stream, q, kc, vc, part_out, part_max, part_sum,
                       d_pos, n_heads, n_kv, max_seq);
    hipLaunchKernelGGL(attention_hm_stage2<128>, dim3(n_heads * (128 / kHmMergeDims)), dim3(kWave), 0, stream,
                       part_out, part_max, part_sum, out, d_pos, n_heads, n_kv);
  } else {
    hipLaunchKernelGGL(attention_hm_mfma_stage1<64>, grid, block, 0, stream, q, kc, vc, part_out, part_max, part_sum,
                       d_pos, n_heads, n_kv, max_seq);
    hipLaunchKernelGGL(attention_hm_stage2<64>, dim3(n_heads * (64 / kHmMergeDims)), dim3(kWave), 0, stream,
                       part_out, part_max, part_sum, out, d_pos, n_heads, n_kv);
  }
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

int launch_kv_store_hm(const __half* k, const __half* v, __half* kc, __half* vc, const int* d_pos, int n_kv,
                       int max_seq, int hd, hipStream_t stream) {
  if (!k || !v || !kc || !vc || !d_pos) return fail(CQ_EINVAL, "kv store (head-major): null pointer");
  if (n_kv <= 0 || hd <= 0 || max_seq <= 0) return fail(CQ_EINVAL, "kv store (head-major): bad shape");
  const int n = n_kv * hd;
  hipLaunchKernelGGL(kv_store_hm_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, k, v, kc, vc, d_pos, n_kv,
                     max_seq, hd);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

}  // namespace cq
