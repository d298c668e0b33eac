// Decode attention and KV store over the reference's head-major cache
// [n_kv][max_seq][head_dim] fp16 (src/model.cu:112-114), for callers that keep
// the reference's layout and its partial buffers at the op level
// (launch_gqa_attention_decode / launch_kv_cache_store,
// include/kernels.cuh:21-47).  The engine's own step uses the MFMA-tiled
// cache of cq_attention.hip; this path exists so that a head-major cache is
// read correctly instead of being misread as tiled.
//
// Stage 1: grid (n_kv, 64 partitions) like kernels.cu:290-324, partition p
// covering keys [p*chunk, min((p+1)*chunk, T)) with chunk = ceil(T/64).  Four
// waves per block; a wave takes 64 keys at a time:
//   * scores: one key per lane, its K row read as 16-byte pieces, dotted with
//     the GQA group's query heads (held in LDS as fp32, read as broadcasts);
//     scores are rounded to fp16 after the 1/sqrt(hd) scale (kernels.cu:171);
//   * online softmax per head over the 64 scores (DPP wave max / sum); P is
//     rounded to fp16 for the PV product, the sum adds the unrounded values
//     (kernels.cu:185-186);
//   * PV: the wave turns to one (hd = 64) or two (hd = 128) dims per lane and
//     walks the 64 V rows, each row read by the whole wave as one contiguous
//     128 / 256-byte line, P broadcast from LDS.
// The four waves merge in LDS and the block writes the partition's
// (max, sum, unnormalised O) at the reference's partial index
// (kv_head * 16 + head) * 64 + partition (kernels.cuh:10-16).
// Stage 2: one block per query head, one thread per dim, log-sum-exp merge
// with 1 / (L + 1e-9) (kernels.cu:222-288).
#include "cq_device.h"
#include "cq_internal.h"

namespace cq {

constexpr int kHmParts = 64;      // ATTN_PARTITIONS (include/config.h:146)
constexpr int kHmSlots = 16;      // PARTIAL_HEAD_SLOTS (include/kernels.cuh:16)
constexpr int kHmWaves = 4;

// Orders this wave's LDS writes before its later LDS reads (lanes read what
// other lanes of the same wave wrote).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int HD>
__global__ __launch_bounds__(kHmWaves * kWave) void attention_hm_stage1(
    const __half* __restrict__ q, const __half* __restrict__ kc, const __half* __restrict__ vc,
    float* __restrict__ part_out, float* __restrict__ part_max, float* __restrict__ part_sum,
    const int* __restrict__ d_pos, int n_heads, int n_kv, int max_seq) {
  constexpr int DPL = HD / kWave;     // dims per lane in the PV phase
  constexpr int NC = HD / 8;          // 16-byte pieces of a row
  const int kvh = blockIdx.x, part = blockIdx.y;
  const int g = n_heads / n_kv;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int T = *d_pos + 1;
  const int chunk = (T + kHmParts - 1) / kHmParts;
  const int t0 = part * chunk, t1 = min(t0 + chunk, T);
  if (t0 >= t1) return;   // block-uniform: no barrier has been reached yet

  __shared__ float qs[kHmSlots][HD];
  __shared__ float ps[kHmWaves][kHmSlots][kWave];
  __shared__ float mw[kHmWaves][kHmSlots], lw[kHmWaves][kHmSlots];
  __shared__ float ow[kHmWaves][kHmSlots][HD];
  for (int i = threadIdx.x; i < g * HD; i += blockDim.x)
    qs[i / HD][i % HD] = (float)q[(size_t)(kvh * g + i / HD) * HD + i % HD];
  __syncthreads();

  const float scale = 1.0f / sqrtf((float)HD);
  const __half* kbase = kc + (size_t)kvh * max_seq * HD;
  const __half* vbase = vc + (size_t)kvh * max_seq * HD;
  float m[kHmSlots], l[kHmSlots], o[kHmSlots][DPL];
#pragma unroll
  for (int h = 0; h < kHmSlots; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[h][e] = 0.f;
  }
  for (int k0 = t0 + wave * kWave; k0 < t1; k0 += kHmWaves * kWave) {
    const int t = k0 + lane;
    const bool valid = t < t1;
    float acc[kHmSlots];
#pragma unroll
    for (int h = 0; h < kHmSlots; ++h) acc[h] = 0.f;
    if (valid) {
      const u4_t* krow = reinterpret_cast<const u4_t*>(kbase + (size_t)t * HD);
#pragma unroll 4
      for (int c = 0; c < NC; ++c) {
        const u4_t w = krow[c];
        float kf[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const h2_t p = as_h2(w[i]);
          kf[2 * i] = (float)p[0];
          kf[2 * i + 1] = (float)p[1];
        }
#pragma unroll
        for (int h = 0; h < kHmSlots; ++h) {
          if (h < g) {
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[h] = fmaf(qs[h][8 * c + i], kf[i], acc[h]);
          }
        }
      }
    }
#pragma unroll
    for (int h = 0; h < kHmSlots; ++h) {
      if (h < g) {
        const float s = valid ? (float)(_Float16)(acc[h] * scale) : -INFINITY;
        const float mn = fmaxf(m[h], wave_max(s));   // finite: lane 0 of the group is valid
        const float f = __expf(m[h] - mn);           // m = -inf on the first group gives 0
        const float p = valid ? __expf(s - mn) : 0.f;
        l[h] = l[h] * f + wave_sum(p);
        m[h] = mn;
        ps[wave][h][lane] = (float)(_Float16)p;
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[h][e] *= f;
      }
    }
    wave_lds_sync();
    const int nk = min(kWave, t1 - k0);
    for (int j = 0; j < nk; ++j) {
      const __half* vrow = vbase + (size_t)(k0 + j) * HD + lane * DPL;
      float vf[DPL];
      if constexpr (DPL == 2) {
        const h2_t p = as_h2(*reinterpret_cast<const uint32_t*>(vrow));
        vf[0] = (float)p[0];
        vf[1] = (float)p[1];
      } else {
        vf[0] = (float)*reinterpret_cast<const _Float16*>(vrow);
      }
#pragma unroll
      for (int h = 0; h < kHmSlots; ++h)
        if (h < g)
#pragma unroll
          for (int e = 0; e < DPL; ++e) o[h][e] = fmaf(ps[wave][h][j], vf[e], o[h][e]);
    }
    wave_lds_sync();   // P is rewritten by the next group
  }
  // merge the four waves
#pragma unroll
  for (int h = 0; h < kHmSlots; ++h) {
    if (h < g) {
      if (lane == 0) {
        mw[wave][h] = m[h];
        lw[wave][h] = l[h];
      }
#pragma unroll
      for (int e = 0; e < DPL; ++e) ow[wave][h][lane * DPL + e] = o[h][e];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < g * HD; i += blockDim.x) {
    const int h = i / HD, d = i % HD;
    float M = -INFINITY;
    for (int w = 0; w < kHmWaves; ++w) M = fmaxf(M, mw[w][h]);
    float L = 0.f, O = 0.f;
    for (int w = 0; w < kHmWaves; ++w) {
      if (mw[w][h] == -INFINITY) continue;   // a wave with no keys in this partition
      const float r = __expf(mw[w][h] - M);
      L += lw[w][h] * r;
      O += ow[w][h][d] * r;
    }
    const size_t slot = (size_t)(kvh * kHmSlots + h) * kHmParts + part;
    part_out[slot * HD + d] = O;
    if (d == 0) {
      part_max[slot] = M;
      part_sum[slot] = L;
    }
  }
}

template <int HD>
__global__ __launch_bounds__(HD) void attention_hm_stage2(const float* __restrict__ part_out,
                                                         const float* __restrict__ part_max,
                                                         const float* __restrict__ part_sum, __half* __restrict__ out,
                                                         const int* __restrict__ d_pos, int n_heads, int n_kv) {
  const int h = blockIdx.x, d = threadIdx.x;
  const int g = n_heads / n_kv;
  const size_t pslot = (size_t)(h / g) * kHmSlots + h % g;
  const int T = *d_pos + 1;
  const int chunk = (T + kHmParts - 1) / kHmParts;
  const int nonempty = (T + chunk - 1) / chunk;
  float M = -1e30f;
  for (int s = 0; s < nonempty; ++s) M = fmaxf(M, part_max[pslot * kHmParts + s]);
  float L = 0.f, O = 0.f;
  for (int s = 0; s < nonempty; ++s) {
    const float r = __expf(part_max[pslot * kHmParts + s] - M);
    L += part_sum[pslot * kHmParts + s] * r;
    O += part_out[(pslot * kHmParts + s) * HD + d] * r;
  }
  out[(size_t)h * HD + d] = (__half)(O * (1.0f / (L + 1e-9f)));
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
  const dim3 grid(n_kv, kHmParts), block(kHmWaves * kWave);
  if (head_dim == 128) {
    hipLaunchKernelGGL(attention_hm_stage1<128>, grid, block, 0, stream, q, kc, vc, part_out, part_max, part_sum,
                       d_pos, n_heads, n_kv, max_seq);
    hipLaunchKernelGGL(attention_hm_stage2<128>, dim3(n_heads), dim3(128), 0, stream, part_out, part_max, part_sum,
                       out, d_pos, n_heads, n_kv);
  } else {
    hipLaunchKernelGGL(attention_hm_stage1<64>, grid, block, 0, stream, q, kc, vc, part_out, part_max, part_sum,
                       d_pos, n_heads, n_kv, max_seq);
    hipLaunchKernelGGL(attention_hm_stage2<64>, dim3(n_heads), dim3(64), 0, stream, part_out, part_max, part_sum,
                       out, d_pos, n_heads, n_kv);
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
