// Op-level C ABI (the reference's launch_* family, include/kernels.cuh) and
// device-memory helpers.
#include "cq_device.h"
#include "cq_internal.h"

#include <vector>

using namespace cq;

static hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

extern "C" int cq_device_count(int32_t* n) {
  if (!n) return fail(CQ_EINVAL, "null argument");
  int c = 0;
  CQ_HIP(hipGetDeviceCount(&c));
  *n = c;
  return CQ_OK;
}
extern "C" int cq_malloc(void** p, size_t bytes) {
  if (!p) return fail(CQ_EINVAL, "null argument");
  if (hipMalloc(p, bytes ? bytes : 1) != hipSuccess) return fail(CQ_ENOMEM, "hipMalloc failed");
  return CQ_OK;
}
extern "C" int cq_free(void* p) {
  if (p) CQ_HIP(hipFree(p));
  return CQ_OK;
}
extern "C" int cq_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  CQ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return CQ_OK;
}
extern "C" int cq_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  CQ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return CQ_OK;
}
extern "C" int cq_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  CQ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
  return CQ_OK;
}
extern "C" int cq_memset(void* p, int value, size_t bytes) {
  CQ_HIP(hipMemset(p, value, bytes));
  return CQ_OK;
}
extern "C" int cq_synchronize(void) {
  CQ_HIP(hipDeviceSynchronize());
  return CQ_OK;
}

extern "C" int cq_embedding_lookup(const void* embed, const int32_t* d_token, void* out, int32_t dim, void* stream) {
  return launch_embedding((const __half*)embed, d_token, (__half*)out, dim, as_stream(stream));
}

extern "C" int cq_rmsnorm(const void* x, const void* w, void* out, int32_t dim, float eps, void* stream) {
  return launch_rmsnorm((const __half*)x, (const __half*)w, (__half*)out, dim, eps, as_stream(stream));
}

extern "C" int cq_gemv(int32_t quant_type, int32_t group_size, const void* W, const void* scale, const void* x, void* y,
                       int32_t rows, int32_t cols, void* stream) {
  GemvArgs a;
  a.mode = GM_STORE; a.quant = quant_type; a.group = group_size; a.x = (const __half*)x;
  a.K = cols; a.N = rows; a.W[0] = W; a.S[0] = (const __half*)scale; a.out[0] = (__half*)y;
  return launch_gemv(a, as_stream(stream));
}

extern "C" int cq_gemv_add(int32_t quant_type, const void* W, const void* scale, const void* input, void* x_inout,
                           int32_t rows, int32_t cols, void* stream) {
  GemvArgs a;
  a.mode = GM_RESID; a.quant = quant_type; a.x = (const __half*)input;
  a.K = cols; a.N = rows; a.W[0] = W; a.S[0] = (const __half*)scale; a.out[0] = (__half*)x_inout;
  return launch_gemv(a, as_stream(stream));
}

extern "C" int cq_fused_attn_block(int32_t quant_type, const void* x, const void* norm_weight, const void* Wq,
                                   const void* Wk, const void* Wv, const void* Sq, const void* Sk, const void* Sv,
                                   const void* bq, const void* bk, const void* bv, void* q_out, void* k_out,
                                   void* v_out, int32_t dim, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                   const int32_t* d_pos, float rope_theta, float eps, void* stream) {
  if (!q_out || !k_out || !v_out) return fail(CQ_EINVAL, "fused_attn_block: null output");
  GemvArgs a;
  a.mode = GM_QKV; a.quant = quant_type; a.x = (const __half*)x; a.norm_w = (const __half*)norm_weight; a.eps = eps;
  a.K = dim; a.N = (n_heads + 2 * n_kv_heads) * head_dim;
  a.W[0] = Wq; a.W[1] = Wk; a.W[2] = Wv;
  a.S[0] = (const __half*)Sq; a.S[1] = (const __half*)Sk; a.S[2] = (const __half*)Sv;
  a.bias[0] = (const __half*)bq; a.bias[1] = (const __half*)bk; a.bias[2] = (const __half*)bv;
  a.out[0] = (__half*)q_out; a.out[1] = (__half*)k_out; a.out[2] = (__half*)v_out;
  a.n_heads = n_heads; a.n_kv = n_kv_heads; a.head_dim = head_dim; a.d_pos = d_pos; a.rope_theta = rope_theta;
  // no table: the kernel evaluates theta^(-2i/hd) itself
  return launch_gemv(a, as_stream(stream));
}

extern "C" int cq_fused_mlp_stage1(int32_t quant_type, const void* x, const void* norm_weight, const void* Wg,
                                   const void* Wu, const void* Sg, const void* Su, void* out, int32_t dim,
                                   int32_t inter_dim, float eps, void* stream) {
  GemvArgs a;
  a.mode = GM_SWIGLU; a.quant = quant_type; a.x = (const __half*)x; a.norm_w = (const __half*)norm_weight; a.eps = eps;
  a.K = dim; a.N = inter_dim; a.W[0] = Wg; a.W[1] = Wu; a.S[0] = (const __half*)Sg; a.S[1] = (const __half*)Su;
  a.out[0] = (__half*)out;
  return launch_gemv(a, as_stream(stream));
}

extern "C" int cq_fused_mlp_stage2(int32_t quant_type, void* x, const void* Wd, const void* Sd, const void* inter,
                                   int32_t dim, int32_t inter_dim, void* stream) {
  return cq_gemv_add(quant_type, Wd, Sd, inter, x, dim, inter_dim, stream);
}

extern "C" int cq_compute_logits(int32_t lm_quant, const void* x, const void* W, const void* scale, void* logits,
                                 int32_t vocab, int32_t dim, void* stream) {
  if (lm_quant != CQ_LMHEAD_FP16 && lm_quant != CQ_LMHEAD_INT8) return fail(CQ_EINVAL, "compute_logits: bad format");
  GemvArgs a;
  a.mode = GM_STORE; a.quant = lm_quant == CQ_LMHEAD_INT8 ? CQ_QUANT_INT8 : CQ_QUANT_FP16; a.x = (const __half*)x;
  a.K = dim; a.N = vocab; a.W[0] = W; a.S[0] = (const __half*)scale; a.out[0] = (__half*)logits;
  return launch_gemv(a, as_stream(stream));
}

namespace cq {
int launch_epoch_bump(uint32_t* d_epoch, hipStream_t stream);
}

// Workspace: [epoch uint32, padded to 256 B][stamp uint32 x vocab]; zero it
// once before the first call.
extern "C" size_t cq_penalty_workspace_bytes(int32_t vocab) { return 256 + (size_t)(vocab > 0 ? vocab : 0) * 4; }

extern "C" int cq_apply_repetition_penalty(void* logits, const int32_t* d_history, const int32_t* d_history_len,
                                           int32_t vocab, float penalty, void* workspace, void* stream) {
  if (!logits || !d_history || !d_history_len || !workspace || vocab <= 0)
    return fail(CQ_EINVAL, "repetition_penalty: bad arguments");
  uint32_t* epoch = (uint32_t*)workspace;
  uint32_t* stamp = (uint32_t*)((char*)workspace + 256);
  const hipStream_t st = as_stream(stream);
  CQ_TRY(launch_epoch_bump(epoch, st));
  CQ_TRY(launch_stamp_history(stamp, d_history, d_history_len, vocab, epoch, st));
  return launch_penalty_apply((__half*)logits, stamp, epoch, vocab, penalty, st);
}

extern "C" size_t cq_argmax_workspace_bytes(int32_t vocab) {
  (void)vocab;
  return kArgmaxBlocks * 8 + 64;
}

extern "C" int cq_argmax(const void* logits, int32_t* d_token_out, int32_t vocab, void* workspace, void* stream) {
  if (!d_token_out) return fail(CQ_EINVAL, "argmax: null output");
  return launch_argmax((const __half*)logits, vocab, (unsigned long long*)workspace, nullptr, d_token_out, nullptr,
                       nullptr, as_stream(stream));
}

extern "C" int cq_rope(void* q, void* k, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const int32_t* d_pos,
                       float rope_theta, void* stream) {
  return launch_rope((__half*)q, (__half*)k, n_heads, n_kv_heads, head_dim, d_pos, rope_theta, as_stream(stream));
}

extern "C" int cq_kv_cache_store(const void* k, const void* v, void* kc, void* vc, const int32_t* d_pos,
                                 int32_t n_kv_heads, int32_t max_seq_len, int32_t head_dim, void* stream) {
  return launch_kv_store((const __half*)k, (const __half*)v, (__half*)kc, (__half*)vc, d_pos, n_kv_heads, max_seq_len,
                         head_dim, as_stream(stream));
}

extern "C" size_t cq_attention_workspace_bytes(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim) {
  if (n_kv_heads <= 0 || head_dim <= 0) return 0;
  return attention_workspace_bytes(n_heads, n_kv_heads, head_dim);
}

extern "C" int cq_gqa_attention_decode(const void* q, const void* kc, const void* vc, void* out, const int32_t* d_pos,
                                       int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                       void* workspace, void* stream) {
  AttnArgs a;
  a.q = (const __half*)q; a.kcache = (const __half*)kc; a.vcache = (const __half*)vc; a.out = (__half*)out;
  a.d_pos = d_pos; a.n_heads = n_heads; a.n_kv = n_kv_heads; a.head_dim = head_dim; a.max_seq = max_seq_len;
  a.workspace = workspace;
  return launch_attention(a, as_stream(stream));
}

extern "C" int cq_kv_cache_store_hm(const void* k, const void* v, void* kc, void* vc, const int32_t* d_pos,
                                    int32_t n_kv_heads, int32_t max_seq_len, int32_t head_dim, void* stream) {
  return launch_kv_store_hm((const __half*)k, (const __half*)v, (__half*)kc, (__half*)vc, d_pos, n_kv_heads,
                            max_seq_len, head_dim, as_stream(stream));
}

extern "C" int cq_gqa_attention_decode_hm(const void* q, const void* kc, const void* vc, void* out,
                                          const int32_t* d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                          int32_t max_seq_len, float* partial_out, float* partial_max,
                                          float* partial_sum, void* stream) {
  return launch_attention_hm((const __half*)q, (const __half*)kc, (const __half*)vc, (__half*)out, d_pos, n_heads,
                             n_kv_heads, head_dim, max_seq_len, partial_out, partial_max, partial_sum,
                             as_stream(stream));
}

static int attention_decode_q(int fmt, const void* q, const void* k_new, const void* v_new, void* k_cache8,
                              void* v_cache8, float* k_scale, float* v_scale, void* out, const int32_t* d_pos,
                              int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t max_seq_len,
                              void* workspace, void* stream) {
  AttnArgs a;
  a.kv_fmt = fmt;
  a.q = (const __half*)q; a.out = (__half*)out;
  a.kcache8 = (int8_t*)k_cache8; a.vcache8 = (int8_t*)v_cache8; a.kscale = k_scale; a.vscale = v_scale;
  a.k_new = (const __half*)k_new; a.v_new = (const __half*)v_new;
  a.d_pos = d_pos; a.n_heads = n_heads; a.n_kv = n_kv_heads; a.head_dim = head_dim; a.max_seq = max_seq_len;
  a.workspace = workspace;
  if (!k_cache8) return fail(CQ_EINVAL, "attention: null cache pointer");
  return launch_attention(a, as_stream(stream));
}

extern "C" int cq_gqa_attention_decode_kv8(const void* q, const void* k_new, const void* v_new, void* k_cache8,
                                           void* v_cache8, float* k_scale, float* v_scale, void* out,
                                           const int32_t* d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                           int32_t max_seq_len, void* workspace, void* stream) {
  return attention_decode_q(CQ_KV_INT8, q, k_new, v_new, k_cache8, v_cache8, k_scale, v_scale, out, d_pos, n_heads,
                            n_kv_heads, head_dim, max_seq_len, workspace, stream);
}

extern "C" int cq_gqa_attention_decode_fp8(const void* q, const void* k_new, const void* v_new, void* k_cache8,
                                           void* v_cache8, float* k_scale, float* v_scale, void* out,
                                           const int32_t* d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                           int32_t max_seq_len, void* workspace, void* stream) {
  return attention_decode_q(CQ_KV_FP8, q, k_new, v_new, k_cache8, v_cache8, k_scale, v_scale, out, d_pos, n_heads,
                            n_kv_heads, head_dim, max_seq_len, workspace, stream);
}

extern "C" int cq_dequantize(int32_t quant_type, int32_t group_size, const void* W, const void* scale, float* out,
                             int32_t rows, int32_t cols, void* stream) {
  return launch_dequant(quant_type, group_size, W, (const __half*)scale, out, rows, cols, as_stream(stream));
}

extern "C" int cq_time_gemv(int32_t quant_type, int32_t group_size, int32_t n_bufs, void* const* W_list,
                            void* const* S_list, const void* x, void* y, int32_t rows, int32_t cols, int32_t iters,
                            double* us_per_launch) {
  if (n_bufs <= 0 || !W_list || iters <= 0 || !us_per_launch) return fail(CQ_EINVAL, "time_gemv: bad arguments");
  hipStream_t st;
  CQ_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  GemvArgs a;
  a.mode = GM_STORE; a.quant = quant_type; a.group = group_size; a.x = (const __half*)x; a.K = cols; a.N = rows;
  a.out[0] = (__half*)y;
  int rc = CQ_OK;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float ms = 0.f;
  auto body = [&]() -> int {
    CQ_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < iters; ++i) {
      a.W[0] = W_list[i % n_bufs];
      a.S[0] = S_list ? (const __half*)S_list[i % n_bufs] : nullptr;
      int r = launch_gemv(a, st);
      if (r != CQ_OK) {
        hipGraph_t dummy;
        hipStreamEndCapture(st, &dummy);
        if (dummy) hipGraphDestroy(dummy);
        return r;
      }
    }
    CQ_HIP(hipStreamEndCapture(st, &g));
    CQ_HIP(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    CQ_HIP(hipGraphLaunch(ge, st));   // warm-up
    CQ_HIP(hipEventCreate(&e0));
    CQ_HIP(hipEventCreate(&e1));
    CQ_HIP(hipEventRecord(e0, st));
    CQ_HIP(hipGraphLaunch(ge, st));
    CQ_HIP(hipEventRecord(e1, st));
    CQ_HIP(hipEventSynchronize(e1));
    CQ_HIP(hipEventElapsedTime(&ms, e0, e1));
    return CQ_OK;
  };
  rc = body();
  if (ge) hipGraphExecDestroy(ge);
  if (g) hipGraphDestroy(g);
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  hipStreamDestroy(st);
  if (rc == CQ_OK) *us_per_launch = (double)ms * 1000.0 / iters;
  return rc;
}

// ------------------------------------------------------------ streaming floor
// A plain streaming read of n_bytes (16-byte nontemporal loads, four per
// thread in flight, four 256-thread blocks per CU striding over the buffer,
// folded into a word so the loads are not removed): the floor a kernel of
// that many bytes meets in a graph chain.  Of the streaming shapes measured
// (one 1024-thread block per CU reading a contiguous range, 512- and
// 256-thread grids, 2 / 4 / 6 / 8 loads in flight, rolling prefetch, plain
// and nontemporal loads) this one was the fastest from 8.5 MB to 554 MB.
// n_bytes 0 launches the same grid with nothing to read (the per-node cost).
namespace {
__global__ __launch_bounds__(256) void stream_read_kernel(const u4_t* p, size_t n16, uint32_t* sink) {
  // grid-stride: iteration i of block b reads 4 x 256 chunks at (i * G + b) * 1024,
  // so at any moment the grid's loads cover one contiguous window of the buffer
  const size_t step = (size_t)gridDim.x * blockDim.x * 4;
  uint32_t acc = 0;
  size_t i = (size_t)blockIdx.x * blockDim.x * 4 + threadIdx.x;
  for (; i + 3 * blockDim.x < n16; i += step) {
    const u4_t a = load_u4_stream(p + i), b = load_u4_stream(p + i + blockDim.x);
    const u4_t c = load_u4_stream(p + i + 2 * blockDim.x), d = load_u4_stream(p + i + 3 * blockDim.x);
    acc += a.x ^ b.y ^ c.z ^ d.w;
  }
  for (; i < n16; i += blockDim.x) acc += load_u4_stream(p + i).x;
  if (acc == 0x9E3779B9u) sink[0] = acc;   // practically never: keeps the loads
}
}  // namespace

// Grid-wide barriers inside one kernel, the alternative to a graph-node
// boundary between dependent stages.  Block b arrives at barrier r by
// publishing r (kind 0: its own flag, one 128-byte line per block, which
// every block then polls, one flag per thread; kind 1: one device-scope
// atomic add to a shared counter, which every block polls until it reaches
// r * blocks; kind 2: its own flag, which only block 0 polls before it
// publishes r in one word that every other block polls; kind 3: kind 2
// with relaxed stores and no acquire fence, i.e. the signalling alone --
// a barrier that orders no other memory, the lower bound).  Every poll loop is bounded: past kBarrierSpins polls the
// block records a time-out and all blocks leave, so the kernel always ends.
namespace {
constexpr int kBarrierSpins = 1 << 22;
constexpr int kFlagStride = 32;   // uint32 per 128-byte line

// polls are relaxed device-scope loads; one acquire fence follows the wait
__device__ __forceinline__ uint32_t ld_poll(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void grid_barrier_kernel(uint32_t* flags, uint32_t* counter, uint32_t* timed_out,
                                                           int kind, int rounds) {
  __shared__ int stop;
  const uint32_t nb = gridDim.x;
  for (int r = 1; r <= rounds; ++r) {
    if (threadIdx.x == 0) {
      if (kind == 3) __hip_atomic_store(flags + blockIdx.x * kFlagStride, (uint32_t)r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else if (kind != 1) __hip_atomic_store(flags + blockIdx.x * kFlagStride, (uint32_t)r, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      else __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      stop = 0;
    }
    __syncthreads();
    int spins = 0;
    if (kind == 0) {
      if (threadIdx.x < nb)
        while (ld_poll(flags + threadIdx.x * kFlagStride) < (uint32_t)r && ++spins < kBarrierSpins) {}
    } else if (kind == 1) {
      if (threadIdx.x == 0)
        while (ld_poll(counter) < (uint32_t)r * nb && ++spins < kBarrierSpins) {}
    } else {
      // block 0 gathers the flags and publishes round r in one word the others poll
      if (blockIdx.x == 0) {
        if (threadIdx.x < nb)
          while (ld_poll(flags + threadIdx.x * kFlagStride) < (uint32_t)r && ++spins < kBarrierSpins) {}
        __syncthreads();
        if (threadIdx.x == 0) {
          if (kind == 3) __hip_atomic_store(counter, (uint32_t)r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else __hip_atomic_store(counter, (uint32_t)r, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else if (threadIdx.x == 0) {
        while (ld_poll(counter) < (uint32_t)r && ++spins < kBarrierSpins) {}
      }
    }
    if (kind != 3) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (spins >= kBarrierSpins) {
      stop = 1;
      __hip_atomic_store(timed_out, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (stop || __hip_atomic_load(timed_out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
  }
}
}  // namespace

extern "C" int cq_time_grid_barrier(int32_t kind, int32_t blocks, int32_t rounds, double* us_per_barrier,
                                    int32_t* timed_out) {
  if (kind < 0 || kind > 3 || rounds <= 0 || !us_per_barrier || !timed_out)
    return fail(CQ_EINVAL, "time_grid_barrier: bad arguments");
  int dev = 0, cus = 0;
  CQ_HIP(hipGetDevice(&dev));
  CQ_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  // one block per CU at most: all blocks resident at once (every block waits for every other)
  if (blocks <= 0 || blocks > cus || blocks > 256) return fail(CQ_EINVAL, "time_grid_barrier: blocks outside [1, CUs]");
  hipStream_t st;
  CQ_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  uint32_t* mem = nullptr;
  hipEvent_t e[4] = {nullptr, nullptr, nullptr, nullptr};
  float ms_full = 0.f, ms_empty = 0.f;
  uint32_t to = 0;
  const size_t flag_words = (size_t)blocks * kFlagStride;
  auto body = [&]() -> int {
    CQ_HIP(hipMalloc(&mem, (flag_words + 64) * sizeof(uint32_t)));
    uint32_t* counter = mem + flag_words;
    uint32_t* tflag = counter + 32;
    for (auto& ev : e) CQ_HIP(hipEventCreate(&ev));
    for (int rep = 0; rep < 2; ++rep) {   // the first pass warms up
      CQ_HIP(hipMemsetAsync(mem, 0, (flag_words + 64) * sizeof(uint32_t), st));
      CQ_HIP(hipEventRecord(e[0], st));
      hipLaunchKernelGGL(grid_barrier_kernel, dim3(blocks), dim3(256), 0, st, mem, counter, tflag, (int)kind, 0);
      CQ_HIP(hipEventRecord(e[1], st));
      CQ_HIP(hipEventRecord(e[2], st));
      hipLaunchKernelGGL(grid_barrier_kernel, dim3(blocks), dim3(256), 0, st, mem, counter, tflag, (int)kind, (int)rounds);
      CQ_HIP(hipEventRecord(e[3], st));
      CQ_HIP(hipGetLastError());
      CQ_HIP(hipEventSynchronize(e[3]));
    }
    CQ_HIP(hipEventElapsedTime(&ms_empty, e[0], e[1]));
    CQ_HIP(hipEventElapsedTime(&ms_full, e[2], e[3]));
    CQ_HIP(hipMemcpy(&to, tflag, sizeof to, hipMemcpyDeviceToHost));
    return CQ_OK;
  };
  const int rc = body();
  for (auto& ev : e)
    if (ev) hipEventDestroy(ev);
  hipStreamSynchronize(st);
  if (mem) hipFree(mem);
  hipStreamDestroy(st);
  if (rc == CQ_OK) {
    *us_per_barrier = (double)(ms_full - ms_empty) * 1000.0 / rounds;
    *timed_out = to ? 1 : 0;
  }
  return rc;
}

extern "C" int cq_time_stream(size_t n_bytes, int32_t n_bufs, void* const* bufs, int32_t iters, double* us_per_launch) {
  if (n_bufs <= 0 || (!bufs && n_bytes) || iters <= 0 || !us_per_launch || n_bytes % 16)
    return fail(CQ_EINVAL, "time_stream: bad arguments");
  hipStream_t st;
  CQ_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  uint32_t* sink = nullptr;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float ms = 0.f;
  int blocks = 256;
  auto body = [&]() -> int {
    int dev = 0;
    CQ_HIP(hipGetDevice(&dev));
    CQ_HIP(hipDeviceGetAttribute(&blocks, hipDeviceAttributeMultiprocessorCount, dev));
    CQ_HIP(hipMalloc(&sink, 64));
    CQ_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < iters; ++i)
      hipLaunchKernelGGL(stream_read_kernel, dim3(4 * blocks), dim3(256), 0, st,
                         n_bytes ? (const u4_t*)bufs[i % n_bufs] : nullptr, n_bytes / 16, sink);
    CQ_HIP(hipStreamEndCapture(st, &g));
    CQ_HIP(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    CQ_HIP(hipGraphLaunch(ge, st));   // warm-up
    CQ_HIP(hipEventCreate(&e0));
    CQ_HIP(hipEventCreate(&e1));
    CQ_HIP(hipEventRecord(e0, st));
    CQ_HIP(hipGraphLaunch(ge, st));
    CQ_HIP(hipEventRecord(e1, st));
    CQ_HIP(hipEventSynchronize(e1));
    CQ_HIP(hipEventElapsedTime(&ms, e0, e1));
    return CQ_OK;
  };
  const int rc = body();
  if (ge) hipGraphExecDestroy(ge);
  if (g) hipGraphDestroy(g);
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  hipStreamSynchronize(st);
  if (sink) hipFree(sink);
  hipStreamDestroy(st);
  if (rc == CQ_OK) *us_per_launch = (double)ms * 1000.0 / iters;
  return rc;
}
