// Small per-token kernels: embedding lookup, stand-alone RMSNorm, KV-cache
// store, repetition penalty and the greedy argmax with its step bookkeeping.
#include "cq_device.h"
#include "cq_internal.h"

namespace cq {

// ------------------------------------------------------------- embedding
// kernels.cu:85-103: copy row *d_token of the fp16 table.
__global__ void embedding_kernel(const u4_t* embed, const int* d_token, u4_t* out, int vec_dim) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < vec_dim) out[i] = embed[(int64_t)(*d_token) * vec_dim + i];
}
int launch_embedding(const __half* embed, const int* d_token, __half* out, int dim, hipStream_t stream) {
  if (dim % 8 || dim <= 0 || !embed || !d_token || !out) return fail(CQ_EINVAL, "embedding: bad arguments");
  const int vec = dim / 8;
  hipLaunchKernelGGL(embedding_kernel, dim3((vec + 255) / 256), dim3(256), 0, stream, (const u4_t*)embed, d_token,
                     (u4_t*)out, vec);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

// --------------------------------------------------------------- rmsnorm
// kernels.cu:689-768: out = half((x * rsqrt(mean(x^2) + half(eps))) * w).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const _Float16* x, const _Float16* w, _Float16* out, int dim,
                                                      float eps) {
  __shared__ float red[16];
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) ss += (float)x[i] * (float)x[i];
  ss = block_sum(ss, red);
  const float inv = rsqrtf(ss / (float)dim + (float)(_Float16)eps);
  for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = (_Float16)(((float)x[i] * inv) * (float)w[i]);
}
int launch_rmsnorm(const __half* x, const __half* w, __half* out, int dim, float eps, hipStream_t stream) {
  if (dim <= 0 || !x || !w || !out) return fail(CQ_EINVAL, "rmsnorm: bad arguments");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, stream, (const _Float16*)x, (const _Float16*)w,
                     (_Float16*)out, dim, eps);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

// -------------------------------------------------------------- kv store
// kernels.cu:326-367, into the tiled layout of cq_common.h.
__global__ void kv_store_kernel(const _Float16* k, const _Float16* v, _Float16* kc, _Float16* vc, const int* d_pos,
                                int n_kv, int max_seq, int hd) {
  const int tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= n_kv * hd) return;
  const int pos = *d_pos, h = tid / hd, d = tid % hd;
  kc[kv_k_offset(h, pos, d, max_seq, hd)] = k[tid];
  vc[kv_v_offset(h, pos, d, max_seq, hd)] = v[tid];
}
int launch_kv_store(const __half* k, const __half* v, __half* kc, __half* vc, const int* d_pos, int n_kv,
                    int max_seq, int hd, hipStream_t stream) {
  if (!k || !v || !kc || !vc || !d_pos || n_kv <= 0 || hd <= 0 || hd % 32 || max_seq % 32)
    return fail(CQ_EINVAL, "kv_cache_store: bad arguments");
  const int n = n_kv * hd;
  hipLaunchKernelGGL(kv_store_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, (const _Float16*)k,
                     (const _Float16*)v, (_Float16*)kc, (_Float16*)vc, d_pos, n_kv, max_seq, hd);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

// ------------------------------------------------------ repetition penalty
// The reference applies l<0 ? l*p : l/p once per history entry, so repeated
// ids race and ids past 4096 entries are skipped (kernels.cu:873-905).  Here
// every distinct id is stamped with the step's epoch and penalised once.
__global__ void stamp_kernel(uint32_t* stamp, const int* hist, const int* d_len, int vocab, const uint32_t* d_epoch) {
  const int n = *d_len;
  const uint32_t ep = *d_epoch;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const int id = hist[i];
    if (id >= 0 && id < vocab) stamp[id] = ep;
  }
}
int launch_stamp_history(uint32_t* stamp, const int* d_history, const int* d_history_len, int vocab,
                         const uint32_t* d_epoch, hipStream_t stream) {
  hipLaunchKernelGGL(stamp_kernel, dim3(64), dim3(256), 0, stream, stamp, d_history, d_history_len, vocab, d_epoch);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}
__global__ void penalty_kernel(_Float16* logits, const uint32_t* stamp, const uint32_t* d_epoch, int vocab,
                               float penalty) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= vocab || stamp[i] != *d_epoch) return;
  const float pen = (float)(_Float16)penalty;
  const float l = (float)logits[i];
  logits[i] = (_Float16)(l < 0.f ? l * pen : l / pen);
}
int launch_penalty_apply(__half* logits, const uint32_t* stamp, const uint32_t* d_epoch, int vocab, float penalty,
                         hipStream_t stream) {
  hipLaunchKernelGGL(penalty_kernel, dim3((vocab + 255) / 256), dim3(256), 0, stream, (_Float16*)logits, stamp,
                     d_epoch, vocab, penalty);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}
__global__ void epoch_bump_kernel(uint32_t* e) { *e += 1u; }
int launch_epoch_bump(uint32_t* d_epoch, hipStream_t stream) {
  hipLaunchKernelGGL(epoch_bump_kernel, dim3(1), dim3(1), 0, stream, d_epoch);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

// ------------------------------------------------------------------- rope
// Stand-alone RoPE (apply_rope_kernel, kernels.cu:370-398): every q and k
// head rotated in place at position *d_pos, one thread per rotation pair.
// The decode step fuses the same rotation into the QKV epilogue.
__global__ __launch_bounds__(256) void rope_kernel(_Float16* q, _Float16* k, int n_heads, int n_kv, int hd,
                                                   const int* d_pos, float theta) {
  const int half = hd / 2;
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (n_heads + n_kv) * half) return;
  const int head = id / half, i = id % half;
  _Float16* v = head < n_heads ? q + (int64_t)head * hd : k + (int64_t)(head - n_heads) * hd;
  float y0 = (float)v[i], y1 = (float)v[i + half];
  rope_rotate(y0, y1, *d_pos, rope_inv_freq_dev(theta, i, hd));
  v[i] = (_Float16)y0;
  v[i + half] = (_Float16)y1;
}

int launch_rope(__half* q, __half* k, int n_heads, int n_kv, int head_dim, const int* d_pos, float theta,
                hipStream_t stream) {
  if (!q || !k || !d_pos || n_heads <= 0 || n_kv <= 0) return fail(CQ_EINVAL, "rope: bad arguments");
  if (head_dim <= 0 || head_dim > kMaxHeadDim || head_dim % 2) return fail(CQ_EINVAL, "rope: bad head_dim");
  const int n = (n_heads + n_kv) * (head_dim / 2);
  hipLaunchKernelGGL(rope_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, (_Float16*)q, (_Float16*)k, n_heads,
                     n_kv, head_dim, d_pos, theta);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

// ----------------------------------------------------------------- argmax
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* red) {
  v = wave_max_u64(v);
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  unsigned long long b = 0ull;
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) b = red[i] > b ? red[i] : b;
  return b;
}

// Stage 1: each block writes its best key; stage 2 (one block) reduces them
// and does the step bookkeeping (kernels.cu:915-950).  Two launches cost
// less here than one launch with a completion ticket and device-scope fences.
// The decode step skips stage 1: the lm_head GEMV writes one key per wave
// (GemvArgs::argmax_out) and stage 2 reduces those.
__global__ __launch_bounds__(256) void argmax_stage1(const _Float16* logits, int vocab,
                                                     unsigned long long* partials) {
  __shared__ unsigned long long red[16];
  unsigned long long best = 0ull;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < vocab; i += gridDim.x * blockDim.x) {
    const unsigned long long k = argmax_key((float)logits[i], i);
    best = k > best ? k : best;
  }
  best = block_max_u64(best, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = best;
}

constexpr int kArgmaxReduceThreads = 1024;
__global__ __launch_bounds__(kArgmaxReduceThreads) void argmax_stage2(const unsigned long long* partials, int n,
                                                                     StepCtl* ctl, int* d_token_out, int* history,
                                                                     int* tokens_out, StepBegin next) {
  __shared__ unsigned long long red[16];
  __shared__ int next_token;
  // The control block is read once, up front, in flight with the keys:
  // nothing else touches it during this launch, and field-by-field reads
  // behind the stores below would each be a dependent memory round trip.
  // all kernel arguments in the first scalar batch
  CQ_PIN(partials); CQ_PIN(n); CQ_PIN(ctl); CQ_PIN(d_token_out); CQ_PIN(history); CQ_PIN(tokens_out);
  CQ_PIN(next.embed); CQ_PIN(next.x); CQ_PIN(next.dim); CQ_PIN(next.stamp);
  // every key of a thread requested before the first is waited for
  constexpr int kPer = 8;
  unsigned long long k[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    // clamped, not branched (a repeated key leaves the maximum unchanged)
    k[j] = partials[min((int)threadIdx.x + j * kArgmaxReduceThreads, n - 1)];
  }
  StepCtl c{};
  if (ctl && threadIdx.x == 0) c = *ctl;
  unsigned long long v = 0ull;
#pragma unroll
  for (int j = 0; j < kPer; ++j) v = k[j] > v ? k[j] : v;
  for (int i = threadIdx.x + kPer * kArgmaxReduceThreads; i < n; i += kArgmaxReduceThreads)
    v = partials[i] > v ? partials[i] : v;
  const unsigned long long b = block_max_u64(v, red);
  if (threadIdx.x == 0) {
    const int token = (int)(~(uint32_t)(b & 0xffffffffu));
    if (d_token_out) *d_token_out = token;
    if (ctl) {
      ctl->sampled = token;
      if (tokens_out) tokens_out[c.step] = token;
      ctl->step = c.step + 1;
      int chained = -1;
      if (c.chain) {
        ctl->token = token;
        ctl->pos = c.pos + 1;
        if (c.history_len < c.max_history) {
          history[c.history_len] = token;
          ctl->history_len = c.history_len + 1;
          // the history only grows within a chained decode, so the epoch
          // stays and only the appended id needs its stamp
          if (next.stamp) next.stamp[token] = c.epoch;
        }
        chained = token;
      }
      next_token = chained;
    }
  }
  if (!next.x) return;
  __syncthreads();
  // the next chained step's embedding row, so that it needs no step_begin
  const int t = next_token;
  if (t < 0) return;
  const int vec_dim = next.dim / 8;
  const u4_t* row = reinterpret_cast<const u4_t*>(next.embed) + (int64_t)t * vec_dim;
  for (int i = threadIdx.x; i < vec_dim; i += kArgmaxReduceThreads) reinterpret_cast<u4_t*>(next.x)[i] = row[i];
}

int launch_argmax_reduce(const unsigned long long* partials, int n, StepCtl* ctl, int* d_token_out, int* history,
                         int* tokens_out, hipStream_t stream, StepBegin next) {
  if (!partials || n <= 0) return fail(CQ_EINVAL, "argmax: bad arguments");
  if (next.x && (!ctl || !next.embed || next.dim <= 0 || next.dim % 8)) return fail(CQ_EINVAL, "argmax: bad step-begin arguments");
  hipLaunchKernelGGL(argmax_stage2, dim3(1), dim3(kArgmaxReduceThreads), 0, stream, partials, n, ctl, d_token_out,
                     history, tokens_out, next);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

int launch_argmax(const __half* logits, int vocab, unsigned long long* partials, StepCtl* ctl, int* d_token_out,
                  int* history, int* tokens_out, hipStream_t stream) {
  if (!logits || vocab <= 0 || !partials) return fail(CQ_EINVAL, "argmax: bad arguments");
  hipLaunchKernelGGL(argmax_stage1, dim3(kArgmaxBlocks), dim3(256), 0, stream, (const _Float16*)logits, vocab,
                     partials);
  return launch_argmax_reduce(partials, kArgmaxBlocks, ctl, d_token_out, history, tokens_out, stream);
}

// ------------------------------------------------------------ step begin
// Embedding of ctl->token into x (block 0) and history stamping with the
// step's epoch (all blocks).  The epoch is set by the host with each new
// history (a fresh value per call), so stale stamps never match.
__global__ __launch_bounds__(256) void step_begin_kernel(const u4_t* embed, const StepCtl* ctl, const int* history,
                                                         uint32_t* stamp, u4_t* x, int vec_dim, int vocab) {
  const int token = ctl->token;
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < vec_dim; i += blockDim.x) x[i] = embed[(int64_t)token * vec_dim + i];
  }
  const int n = ctl->history_len;
  const uint32_t ep = ctl->epoch;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const int id = history[i];
    if (id >= 0 && id < vocab) stamp[id] = ep;
  }
}
int launch_step_begin(const __half* embed, StepCtl* ctl, const int* history, uint32_t* stamp, __half* x, int dim,
                      int vocab, hipStream_t stream) {
  hipLaunchKernelGGL(step_begin_kernel, dim3(32), dim3(256), 0, stream, (const u4_t*)embed, ctl, history, stamp,
                     (u4_t*)x, dim / 8, vocab);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

}  // namespace cq
