// Decode engine: device weights (file load or on-device synthesis), the
// decode state and the HIP-graph-recorded decode step.
//
// Reference: src/load_weights.cpp:36-199 (loader), src/model.cu:5-223
// (state, step body, graph capture and replay).
#include "cq_device.h"
#include "cq_format.h"
#include "cq_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

using namespace cq;

struct LayerW {
  __half* in_norm = nullptr;
  __half* post_norm = nullptr;
  __half *bq = nullptr, *bk = nullptr, *bv = nullptr;
  void *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr, *wg = nullptr, *wu = nullptr, *wd = nullptr;
  __half *sq = nullptr, *sk = nullptr, *sv = nullptr, *so = nullptr, *sg = nullptr, *su = nullptr, *sd = nullptr;
};

struct cq_weights {
  cq_config cfg{};
  char* arena = nullptr;
  size_t arena_bytes = 0;
  __half* embed = nullptr;
  __half* final_norm = nullptr;
  void* lm_head = nullptr;        // fp16 [V][d] (possibly == embed) or int8 [V][d]
  __half* lm_head_scale = nullptr;
  std::vector<LayerW> layers;
  // per tensor placement in the arena, in file order
  struct Slot { TensorSpec spec; size_t w_off, s_off; };
  std::vector<Slot> slots;
  // exporter-layout (row-major) copy of every layer's Wo and its scales, made
  // on the first cq_weights_wo_rows call; per layer wo_rows_stride bytes
  char* wo_rows = nullptr;
  size_t wo_rows_stride = 0, wo_rows_wbytes = 0;
};

namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Place every tensor in one device arena and wire the pointers.
int weights_layout(cq_weights* w) {
  size_t off = 0;
  for (const auto& t : tensor_list(w->cfg)) {
    cq_weights::Slot s{t, off, 0};
    off = align_up(off + (size_t)t.weight_bytes);
    if (t.scale_bytes) {
      s.s_off = off;
      off = align_up(off + (size_t)t.scale_bytes);
    }
    w->slots.push_back(s);
  }
  w->arena_bytes = off;
  hipError_t e = hipMalloc(&w->arena, off);
  if (e != hipSuccess) return fail(CQ_ENOMEM, std::string("weights: hipMalloc of ") + std::to_string(off) + " bytes failed");
  w->layers.assign(w->cfg.n_layers, LayerW{});
  for (const auto& s : w->slots) {
    void* p = w->arena + s.w_off;
    __half* sc = s.spec.scale_bytes ? reinterpret_cast<__half*>(w->arena + s.s_off) : nullptr;
    __half* hp = reinterpret_cast<__half*>(p);
    LayerW* L = s.spec.layer >= 0 ? &w->layers[s.spec.layer] : nullptr;
    switch (s.spec.kind) {
      case TK_EMBED: w->embed = hp; break;
      case TK_FINAL_NORM: w->final_norm = hp; break;
      case TK_LM_HEAD: w->lm_head = p; w->lm_head_scale = sc; break;
      case TK_IN_NORM: L->in_norm = hp; break;
      case TK_POST_NORM: L->post_norm = hp; break;
      case TK_WQ: L->wq = p; L->sq = sc; break;
      case TK_BQ: L->bq = hp; break;
      case TK_WK: L->wk = p; L->sk = sc; break;
      case TK_BK: L->bk = hp; break;
      case TK_WV: L->wv = p; L->sv = sc; break;
      case TK_BV: L->bv = hp; break;
      case TK_WO: L->wo = p; L->so = sc; break;
      case TK_WG: L->wg = p; L->sg = sc; break;
      case TK_WU: L->wu = p; L->su = sc; break;
      case TK_WD: L->wd = p; L->sd = sc; break;
    }
  }
  if (!w->lm_head) w->lm_head = w->embed;   // tied (load_weights.cpp:159)
  return CQ_OK;
}

// The O-projections into the 128-column panel layout the decode's merged
// O-projection streams contiguously (wo_to_panels); done once, after the
// weights are in the arena, whatever filled it.
int weights_panelize(cq_weights* w) {
  const cq_config& c = w->cfg;
  const int qd = c.n_heads * c.head_dim;
  const int epc = c.quant_type == CQ_QUANT_INT4 ? 32 : c.quant_type == CQ_QUANT_INT8 ? 16 : 8;
  void* tmp = nullptr;
  if (hipMalloc(&tmp, (size_t)c.dim * (qd / epc) * 16) != hipSuccess) return fail(CQ_ENOMEM, "weights: panel staging allocation failed");
  int rc = CQ_OK;
  for (int l = 0; l < c.n_layers && rc == CQ_OK; ++l)
    rc = wo_to_panels(c.quant_type, w->layers[l].wo, w->layers[l].so, c.dim, qd, tmp, nullptr);
  const hipError_t e = hipStreamSynchronize(nullptr);
  hipFree(tmp);
  if (rc == CQ_OK && e != hipSuccess) rc = fail(CQ_EHIP, std::string("weights: panel conversion: ") + hipGetErrorString(e));
  return rc;
}

// ------------------------------------------------------ on-device synthesis
__global__ void synth_half_kernel(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream, float mul, float mean) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = synth_half(seed, stream, (uint64_t)i, mul, mean);
}

// One thread per (row, group of 128): generate, quantize as
// export_weights.py:123-205 (fp32 scale for the division, fp16 stored scale).
__global__ void synth_quant_kernel(uint8_t* q, uint16_t* s, int64_t rows, int64_t cols, int quant, uint64_t seed,
                                   uint64_t stream, float mul) {
  const int64_t ng = cols / kGroup;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * ng) return;
  const int64_t r = id / ng, gi = id % ng;
  const uint64_t base = (uint64_t)(r * cols + gi * kGroup);
  const float qmax = quant == CQ_QUANT_INT4 ? 7.0f : 127.0f;
  float mx = 0.f;
  for (int i = 0; i < kGroup; ++i) mx = fmaxf(mx, fabsf(h2f_bits(synth_half(seed, stream, base + i, mul, 0.f))));
  const float sc = __fdiv_rn(mx, qmax);
  const float safe = sc > 0.f ? sc : 1.0f;
  s[id] = f2h_bits(sc);
  if (quant == CQ_QUANT_INT8) {
    int8_t* qr = reinterpret_cast<int8_t*>(q) + r * cols + gi * kGroup;
    for (int i = 0; i < kGroup; ++i) {
      float v = rintf(__fdiv_rn(h2f_bits(synth_half(seed, stream, base + i, mul, 0.f)), safe));
      qr[i] = (int8_t)fminf(fmaxf(v, -qmax), qmax);
    }
  } else {
    uint8_t* qr = q + r * (cols / 2) + gi * (kGroup / 2);
    for (int i = 0; i < kGroup; i += 2) {
      float v0 = rintf(__fdiv_rn(h2f_bits(synth_half(seed, stream, base + i, mul, 0.f)), safe));
      float v1 = rintf(__fdiv_rn(h2f_bits(synth_half(seed, stream, base + i + 1, mul, 0.f)), safe));
      const int q0 = (int)fminf(fmaxf(v0, -qmax), qmax), q1 = (int)fminf(fmaxf(v1, -qmax), qmax);
      qr[i / 2] = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
    }
  }
}

int synth_device(cq_weights* w, uint64_t seed) {
  const float mul = synth_mul(kWeightSigma);
  for (const auto& s : w->slots) {
    const TensorSpec& t = s.spec;
    const uint64_t stream = tensor_stream(t.layer, t.kind);
    if (t.quant == CQ_QUANT_FP16) {
      const int64_t n = t.rows * t.cols;
      const int blocks = (int)std::min<int64_t>((n + 255) / 256, 65536);
      hipLaunchKernelGGL(synth_half_kernel, dim3(blocks), dim3(256), 0, 0, (uint16_t*)(w->arena + s.w_off), n, seed,
                         stream, mul, kind_mean(t.kind));
    } else {
      const int64_t n = t.rows * (t.cols / kGroup);
      hipLaunchKernelGGL(synth_quant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, 0,
                         (uint8_t*)(w->arena + s.w_off), (uint16_t*)(w->arena + s.s_off), t.rows, t.cols, t.quant,
                         seed, stream, mul);
    }
    CQ_HIP(hipGetLastError());
  }
  CQ_HIP(hipDeviceSynchronize());
  return CQ_OK;
}

}  // namespace

// ====================================================================== state
struct cq_state {
  cq_config cfg{};
  const cq_weights* w = nullptr;
  hipStream_t stream = nullptr;
  char* arena = nullptr;
  __half *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *inter = nullptr, *logits = nullptr;
  __half *kcache = nullptr, *vcache = nullptr;
  size_t layer_kv_halves = 0;       // K (or V) elements of one layer: n_kv * max_seq * head_dim
  int kv_dtype = CQ_KV_FP16;        // CQ_KV_INT8 / CQ_KV_FP8: kcache / vcache hold 1-byte codes, scales below
  float *kscale = nullptr, *vscale = nullptr;   // [layer][kv_head][max_seq] (quantized cache)
  void* attn_ws = nullptr;
  long long* oacc = nullptr;   // [dim] O-projection sum, 64-bit fixed point (2^-32), zero between layers
  __half* xh = nullptr;        // [dim] residual stream after the attention block (h)
  unsigned long long* argmax_ws = nullptr;
  StepCtl* ctl = nullptr;
  int* history = nullptr;
  int* tokens_dev = nullptr;
  uint32_t* stamp = nullptr;
  double* rope_inv_freq = nullptr;   // [head_dim/2]
  int* host_pinned = nullptr;     // staging for the per-step control words
  uint32_t epoch = 1u;            // penalty epoch of the last set_ctl
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph_run = nullptr;       // kStepsPerRun chained steps (cq_decode)
  hipGraphExec_t exec_run = nullptr;
  int attn_mode = CQ_ATTN_SPLIT;        // cq_state_set_attention_mode
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double last_us = 0.0;
  double last_prefill_us = 0.0;
  // batched-prefill workspace, allocated on the first cq_prefill
  char* pf_arena = nullptr;
  __half *pf_x = nullptr, *pf_a = nullptr, *pf_q = nullptr, *pf_ao = nullptr, *pf_inter = nullptr;
  float* pf_inv = nullptr;
  float* pf_part = nullptr;   // split-K partials of the prefill GEMMs
  int* pf_tokens = nullptr;
  int* pf_tokens_host = nullptr;   // pinned staging of a chunk's ids
  hipEvent_t pf_copied = nullptr;  // the staging buffer's last upload has completed
};

namespace {

int layer_gemvs(const cq_state* s, int l, GemvArgs* qkv, GemvArgs* mlp1, GemvArgs* mlp2) {
  const cq_config& c = s->cfg;
  const LayerW& L = s->w->layers[l];
  const int qd = c.n_heads * c.head_dim;
  const bool kv8 = s->kv_dtype != CQ_KV_FP16;
  __half* kc = kv8 ? nullptr : s->kcache + (size_t)l * s->layer_kv_halves;
  __half* vc = kv8 ? nullptr : s->vcache + (size_t)l * s->layer_kv_halves;
  if (qkv) {
    GemvArgs a;
    a.mode = GM_QKV; a.quant = c.quant_type; a.x = s->x; a.norm_w = L.in_norm; a.eps = c.norm_eps;
    a.K = c.dim; a.N = qd + 2 * c.n_kv_heads * c.head_dim;
    a.W[0] = L.wq; a.W[1] = L.wk; a.W[2] = L.wv; a.S[0] = L.sq; a.S[1] = L.sk; a.S[2] = L.sv;
    a.bias[0] = L.bq; a.bias[1] = L.bk; a.bias[2] = L.bv;
    a.out[0] = s->q;
    if (kv8) { a.out[1] = s->k; a.out[2] = s->v; }   // quantized into the cache by the attention kernel
    a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = c.head_dim; a.d_pos = &s->ctl->pos;
    a.rope_theta = c.rope_theta; a.rope_inv_freq = s->rope_inv_freq;
    a.kcache = kc; a.vcache = vc; a.max_seq = c.max_seq_len;
    *qkv = a;
  }
  if (mlp1) {
    GemvArgs a;
    a.mode = GM_SWIGLU; a.quant = c.quant_type; a.x = s->x; a.norm_w = L.post_norm; a.eps = c.norm_eps;
    a.K = c.dim; a.N = c.intermediate_size;
    a.W[0] = L.wg; a.W[1] = L.wu; a.S[0] = L.sg; a.S[1] = L.su; a.out[0] = s->inter;
    *mlp1 = a;
  }
  if (mlp2) {
    GemvArgs a;
    a.mode = GM_RESID; a.quant = c.quant_type; a.x = s->inter; a.K = c.intermediate_size; a.N = c.dim;
    a.W[0] = L.wd; a.S[0] = L.sd; a.out[0] = s->x;
    *mlp2 = a;
  }
  return CQ_OK;
}

AttnArgs layer_attn(const cq_state* s, int l) {
  const cq_config& c = s->cfg;
  AttnArgs a;
  a.q = s->q;
  if (s->kv_dtype != CQ_KV_FP16) {
    const size_t ls = (size_t)l * c.n_kv_heads * c.max_seq_len;
    a.kv_fmt = s->kv_dtype;
    a.kcache8 = reinterpret_cast<int8_t*>(s->kcache) + (size_t)l * s->layer_kv_halves;
    a.vcache8 = reinterpret_cast<int8_t*>(s->vcache) + (size_t)l * s->layer_kv_halves;
    a.kscale = s->kscale + ls;
    a.vscale = s->vscale + ls;
    a.k_new = s->k;
    a.v_new = s->v;
  } else {
    a.kcache = s->kcache + (size_t)l * s->layer_kv_halves;
    a.vcache = s->vcache + (size_t)l * s->layer_kv_halves;
  }
  a.out = s->xb;
  a.d_pos = &s->ctl->pos;
  a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = c.head_dim; a.max_seq = c.max_seq_len;
  a.workspace = s->attn_ws;
  return a;
}

GemvArgs lm_head_gemv(const cq_state* s) {
  const cq_config& c = s->cfg;
  GemvArgs a;
  a.mode = GM_STORE;
  a.quant = c.lm_head_fmt == CQ_LMHEAD_INT8 ? CQ_QUANT_INT8 : CQ_QUANT_FP16;
  a.x = s->x; a.norm_w = s->w->final_norm; a.eps = c.norm_eps;
  a.K = c.dim; a.N = c.vocab_size;
  a.W[0] = s->w->lm_head; a.S[0] = s->w->lm_head_scale; a.out[0] = s->logits;
  a.stamp = s->stamp; a.d_epoch = &s->ctl->epoch; a.penalty = c.repetition_penalty;
  return a;
}

// The layer's O-projection as one launch with the attention merge
// (cq_omerge.hip): the head contributions go to s->oacc.
OMergeArgs layer_omerge(const cq_state* s, int l) {
  const cq_config& c = s->cfg;
  OMergeArgs a;
  a.workspace = s->attn_ws; a.attn = s->xb;
  a.W = s->w->layers[l].wo; a.S = s->w->layers[l].so; a.acc = s->oacc; a.d_pos = &s->ctl->pos;
  a.quant = c.quant_type; a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = c.head_dim;
  a.K = c.n_heads * c.head_dim; a.N = c.dim; a.Pmax = attention_max_parts(c.n_kv_heads);
  return a;
}

// The MLP GEMVs of the fused step: gate/up first forms h = half(x + oacc)
// (also into s->xh), down adds to h and clears oacc for the next layer.
void fused_mlp(const cq_state* s, GemvArgs* m1, GemvArgs* m2) {
  m1->x_acc = s->oacc; m1->x_out = s->xh;
  m2->resid = s->xh; m2->zero = s->oacc; m2->zero_n = s->cfg.dim;
}

// One decoder layer of the step (src/model.cu:96-176) in 5 launches:
// RMSNorm+QKV+bias+RoPE+KV store | attention stage 1 | merge+O-proj |
// h = x + O, RMSNorm+gate/up+SwiGLU | down + residual.
int layer_step(cq_state* s, int l, hipStream_t st) {
  GemvArgs qkv, m1, m2;
  layer_gemvs(s, l, &qkv, &m1, &m2);
  fused_mlp(s, &m1, &m2);
  CQ_TRY(launch_gemv(qkv, st));
  if (s->attn_mode == CQ_ATTN_WHOLE_CONTEXT) {
    CQ_TRY(launch_attn_oproj(layer_attn(s, l), layer_omerge(s, l), st));
  } else {
    CQ_TRY(launch_attention_stage1(layer_attn(s, l), st));
    CQ_TRY(launch_omerge(layer_omerge(s, l), st));
  }
  CQ_TRY(launch_gemv(m1, st));
  CQ_TRY(launch_gemv(m2, st));
  return CQ_OK;
}

// The decode step (src/model.cu:76-181), 5 launches per layer + 3:
//   step_begin (embedding + penalty stamps)
//   per layer: layer_step (5 launches)
//   final RMSNorm+lm_head+penalty | argmax (+ on-device step chaining)
int step_body(cq_state* s, bool begin = true) {
  const cq_config& c = s->cfg;
  hipStream_t st = s->stream;
  if (begin) CQ_TRY(launch_step_begin(s->w->embed, s->ctl, s->history, s->stamp, s->x, c.dim, c.vocab_size, st));
  for (int l = 0; l < c.n_layers; ++l) CQ_TRY(layer_step(s, l, st));
  GemvArgs lm = lm_head_gemv(s);
  lm.argmax_out = s->argmax_ws;   // one key per wave, reduced below
  CQ_TRY(launch_gemv(lm, st));
  StepBegin next;   // in a chained decode: the next step's embedding row and its new stamp
  next.embed = s->w->embed; next.x = s->x; next.dim = c.dim; next.stamp = s->stamp;
  CQ_TRY(launch_argmax_reduce(s->argmax_ws, kArgmaxPartials, s->ctl, nullptr, s->history, s->tokens_dev, st, next));
  return CQ_OK;
}

// Steps recorded back to back in the chained-decode graph: one graph launch
// per kStepsPerRun tokens instead of one per token.
constexpr int kStepsPerRun = 8;

int ensure_run_graph(cq_state* s) {
  if (s->exec_run) return CQ_OK;
  if (!s->w) return fail(CQ_EINVAL, "no weights bound to the state (pass them to cq_forward_ex)");
  CQ_HIP(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
  int rc = CQ_OK;
  // steps after the first take their prologue from the previous step's argmax
  for (int i = 0; i < kStepsPerRun && rc == CQ_OK; ++i) rc = step_body(s, i == 0);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(s->stream, &g);
  if (rc != CQ_OK) {
    if (g) hipGraphDestroy(g);
    return rc;
  }
  CQ_HIP(e);
  s->graph_run = g;
  CQ_HIP(hipGraphInstantiate(&s->exec_run, g, nullptr, nullptr, 0));
  return CQ_OK;
}

int ensure_graph(cq_state* s) {
  if (s->exec) return CQ_OK;
  if (!s->w) return fail(CQ_EINVAL, "no weights bound to the state (pass them to cq_forward_ex)");
  CQ_HIP(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
  const int rc = step_body(s);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(s->stream, &g);
  if (rc != CQ_OK) {
    if (g) hipGraphDestroy(g);
    return rc;
  }
  CQ_HIP(e);
  s->graph = g;
  CQ_HIP(hipGraphInstantiate(&s->exec, g, nullptr, nullptr, 0));
  return CQ_OK;
}

// Writes the control words: token, pos, history_len, chain, step, and a new
// penalty epoch for the new history (stamps of earlier calls never match it).
int set_ctl(cq_state* s, int token, int pos, const int32_t* history, int history_len, int chain,
            hipStream_t st = nullptr) {
  if (!st) st = s->stream;
  if (++s->epoch == 0u) s->epoch = 1u;   // stamps start at 0
  StepCtl* h = reinterpret_cast<StepCtl*>(s->host_pinned);
  h->token = token; h->pos = pos; h->history_len = history_len; h->chain = chain; h->step = 0;
  h->sampled = -1; h->max_history = s->cfg.max_seq_len; h->epoch = s->epoch;
  CQ_HIP(hipMemcpyAsync(s->ctl, h, sizeof(StepCtl), hipMemcpyHostToDevice, st));
  if (history_len > 0) {
    CQ_HIP(hipMemcpyAsync(s->history, history, (size_t)history_len * sizeof(int), hipMemcpyHostToDevice, st));
  }
  return CQ_OK;
}

// Binds `w` to the state (deferred binding of a state made without weights,
// or a switch to another weight set of the same shape).  The recorded step
// graph holds the old weight pointers, so it is dropped and recorded again
// on the next step.
int drop_graphs(cq_state* s) {
  if (s->exec) {
    CQ_HIP(hipStreamSynchronize(s->stream));
    hipGraphExecDestroy(s->exec);
    s->exec = nullptr;
  }
  if (s->graph) {
    hipGraphDestroy(s->graph);
    s->graph = nullptr;
  }
  if (s->exec_run) {
    hipGraphExecDestroy(s->exec_run);
    s->exec_run = nullptr;
  }
  if (s->graph_run) {
    hipGraphDestroy(s->graph_run);
    s->graph_run = nullptr;
  }
  return CQ_OK;
}

int bind_weights(cq_state* s, const cq_weights* w) {
  if (!w || w == s->w) return CQ_OK;
  if (std::memcmp(&s->cfg, &w->cfg, offsetof(cq_config, norm_eps)) != 0)
    return fail(CQ_EINVAL, "forward: the weights do not match the state's config");
  CQ_TRY(drop_graphs(s));
  s->w = w;
  return CQ_OK;
}

int check_step_args(const cq_state* s, int token, int pos, const int32_t* history, int history_len) {
  if (pos < 0 || pos >= s->cfg.max_seq_len) return fail(CQ_ERANGE, "position outside [0, max_seq_len)");
  if (token < 0 || token >= s->cfg.vocab_size) return fail(CQ_ERANGE, "token outside the vocabulary");
  if (history_len < 0 || history_len > s->cfg.max_seq_len) return fail(CQ_ERANGE, "history_len outside [0, max_seq_len]");
  if (history_len > 0 && !history) return fail(CQ_EINVAL, "null history with history_len > 0");
  return CQ_OK;
}

__global__ void fill_kv_kernel(__half* kc, __half* vc, int n_layers, int n_kv, int n_pos, int max_seq, int hd,
                               uint64_t seed, float mul) {
  const int64_t per_head = (int64_t)n_pos * hd;
  const int64_t total = (int64_t)n_layers * n_kv * per_head;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = i % per_head;
    const int lh = (int)(i / per_head);
    const int l = lh / n_kv, h = lh % n_kv;
    const int t = (int)(e / hd), d = (int)(e % hd);
    const size_t lo = (size_t)l * n_kv * max_seq * hd;
    kc[lo + kv_k_offset(h, t, d, max_seq, hd)] = __ushort_as_half(synth_half(seed, kv_stream(l, h, 0), e, mul, 0.f));
    vc[lo + kv_v_offset(h, t, d, max_seq, hd)] = __ushort_as_half(synth_half(seed, kv_stream(l, h, 1), e, mul, 0.f));
  }
}

// Quantized cache: one thread per (layer, kv head, position) row of K or V:
// the generator's fp16 values, quantized with s = max|x| / code max and q =
// the code of x / s (int8: rint clamped to +-127; E4M3: round to nearest even).
__device__ __forceinline__ int8_t quant_code(int fmt, float v) {
  return fmt == CQ_KV_FP8 ? (int8_t)e4m3_bits(v) : (int8_t)fminf(127.f, fmaxf(-127.f, rintf(v)));
}
CQ_HD float code_max(int fmt) { return fmt == CQ_KV_FP8 ? 448.0f : 127.0f; }

__global__ void fill_kv8_kernel(int fmt, int8_t* kc, int8_t* vc, float* ks, float* vs, int n_layers, int n_kv,
                                int n_pos, int max_seq, int hd, uint64_t seed, float mul) {
  const int64_t rows = (int64_t)n_layers * n_kv * n_pos * 2;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (int64_t)gridDim.x * blockDim.x) {
    const int kind = (int)(r & 1);
    const int64_t rr = r >> 1;
    const int t = (int)(rr % n_pos);
    const int lh = (int)(rr / n_pos);
    const int l = lh / n_kv, h = lh % n_kv;
    const uint64_t st = kv_stream(l, h, kind);
    float amax = 0.f;
    for (int d = 0; d < hd; ++d)
      amax = fmaxf(amax, fabsf(h2f_bits(synth_half(seed, st, (uint64_t)t * hd + d, mul, 0.f))));
    const float sc = amax / code_max(fmt);
    const size_t lo = (size_t)l * n_kv * max_seq * hd;
    int8_t* c = kind ? vc : kc;
    for (int d = 0; d < hd; ++d) {
      const float x = h2f_bits(synth_half(seed, st, (uint64_t)t * hd + d, mul, 0.f));
      const int8_t q = sc == 0.f ? (int8_t)0 : quant_code(fmt, x / sc);
      c[lo + (kind ? kv8_v_offset(h, t, d, max_seq, hd) : kv8_k_offset(h, t, d, max_seq, hd))] = q;
    }
    (kind ? vs : ks)[((size_t)l * n_kv + h) * max_seq + t] = sc;
  }
}

// The same quantization on the host (cq_state_kv_write of a quantized cache).
void quant_row8_host(int fmt, const uint16_t* x, int n, int8_t* q, float* s) {
  float amax = 0.f;
  for (int i = 0; i < n; ++i) amax = std::max(amax, std::fabs(h2f_bits(x[i])));
  const float sc = amax / code_max(fmt);
  *s = sc;
  for (int i = 0; i < n; ++i) {
    const float v = sc == 0.f ? 0.f : h2f_bits(x[i]) / sc;
    q[i] = sc == 0.f ? (int8_t)0
                     : fmt == CQ_KV_FP8 ? (int8_t)e4m3_bits(v) : (int8_t)std::max(-127.f, std::min(127.f, std::nearbyint(v)));
  }
}

// Value of one stored code (before its row scale).
float code_value(int fmt, int8_t b) { return fmt == CQ_KV_FP8 ? e4m3_value((uint8_t)b) : (float)b; }

}  // namespace

// ===================================================================== C ABI
extern "C" int cq_load_weights(const char* path, const cq_config* expect, cq_config* cfg_out, cq_weights** out) {
  if (!path || !out) return fail(CQ_EINVAL, "load_weights: null argument");
  cq_config c{};
  CQ_TRY(cq_read_header(path, &c));
  if (expect) {
    // load_weights.cpp:62-84: dims and quant type must match the expected config
    if (c.vocab_size != expect->vocab_size || c.dim != expect->dim || c.intermediate_size != expect->intermediate_size ||
        c.n_layers != expect->n_layers || c.n_heads != expect->n_heads || c.n_kv_heads != expect->n_kv_heads ||
        c.head_dim != expect->head_dim)
      return fail(CQ_EFORMAT, "binary header dimensions do not match the expected config");
    if (c.quant_type != expect->quant_type) return fail(CQ_EFORMAT, "quantization mismatch between file and expected config");
  }
  std::unique_ptr<cq_weights> w(new cq_weights);
  w->cfg = c;
  CQ_TRY(weights_layout(w.get()));
  FILE* f = std::fopen(path, "rb");
  if (!f) {
    hipFree(w->arena);
    return fail(CQ_EIO, std::string("cannot open weight file: ") + path);
  }
  std::fseek(f, 256, SEEK_SET);
  const size_t kChunk = 64u << 20;
  void* staging = nullptr;
  if (hipHostMalloc(&staging, kChunk, hipHostMallocDefault) != hipSuccess) {
    std::fclose(f);
    hipFree(w->arena);
    return fail(CQ_ENOMEM, "load_weights: pinned staging allocation failed");
  }
  int rc = CQ_OK;
  auto copy_segment = [&](size_t dst_off, int64_t bytes) -> int {
    int64_t left = bytes;
    size_t at = dst_off;
    while (left > 0) {
      const size_t n = (size_t)std::min<int64_t>(left, (int64_t)kChunk);
      if (std::fread(staging, 1, n, f) != n) return fail(CQ_EIO, "unexpected end of file while reading tensor data");
      if (hipMemcpy(w->arena + at, staging, n, hipMemcpyHostToDevice) != hipSuccess)
        return fail(CQ_EHIP, "load_weights: hipMemcpy failed");
      at += n;
      left -= (int64_t)n;
    }
    return CQ_OK;
  };
  for (const auto& s : w->slots) {
    rc = copy_segment(s.w_off, s.spec.weight_bytes);
    if (rc == CQ_OK && s.spec.scale_bytes) rc = copy_segment(s.s_off, s.spec.scale_bytes);
    if (rc != CQ_OK) break;
  }
  std::fclose(f);
  hipHostFree(staging);
  if (rc == CQ_OK) rc = weights_panelize(w.get());
  if (rc != CQ_OK) {
    hipFree(w->arena);
    return rc;
  }
  if (cfg_out) *cfg_out = c;
  *out = w.release();
  return CQ_OK;
}

extern "C" int cq_synth_weights(const cq_config* cfg, uint64_t seed, cq_weights** out) {
  if (!cfg || !out) return fail(CQ_EINVAL, "synth_weights: null argument");
  CQ_TRY(validate_config(*cfg));
  std::unique_ptr<cq_weights> w(new cq_weights);
  w->cfg = *cfg;
  CQ_TRY(weights_layout(w.get()));
  int rc = synth_device(w.get(), seed);
  if (rc == CQ_OK) rc = weights_panelize(w.get());
  if (rc != CQ_OK) {
    hipFree(w->arena);
    return rc;
  }
  *out = w.release();
  return CQ_OK;
}

extern "C" int cq_free_weights(cq_weights* w) {
  if (!w) return CQ_OK;
  if (w->wo_rows) CQ_HIP(hipFree(w->wo_rows));
  if (w->arena) CQ_HIP(hipFree(w->arena));
  delete w;
  return CQ_OK;
}

extern "C" int cq_weights_tensor(const cq_weights* w, const char* name, int32_t layer, void** dptr, size_t* bytes) {
  if (!w || !name || !dptr) return fail(CQ_EINVAL, "weights_tensor: null argument");
  struct N { const char* n; int kind; bool scale; };
  static const N names[] = {{"embed", TK_EMBED, false}, {"final_norm", TK_FINAL_NORM, false},
                            {"lm_head", TK_LM_HEAD, false}, {"lm_head_scale", TK_LM_HEAD, true},
                            {"in_norm", TK_IN_NORM, false}, {"wq", TK_WQ, false}, {"sq", TK_WQ, true},
                            {"bq", TK_BQ, false}, {"wk", TK_WK, false}, {"sk", TK_WK, true}, {"bk", TK_BK, false},
                            {"wv", TK_WV, false}, {"sv", TK_WV, true}, {"bv", TK_BV, false}, {"wo", TK_WO, false},
                            {"so", TK_WO, true}, {"post_norm", TK_POST_NORM, false}, {"wg", TK_WG, false},
                            {"sg", TK_WG, true}, {"wu", TK_WU, false}, {"su", TK_WU, true}, {"wd", TK_WD, false},
                            {"sd", TK_WD, true}};
  for (const auto& n : names) {
    if (std::strcmp(n.n, name)) continue;
    for (const auto& s : w->slots) {
      if (s.spec.kind != n.kind || (s.spec.layer >= 0 && s.spec.layer != layer)) continue;
      if (n.scale && !s.spec.scale_bytes) return fail(CQ_EINVAL, "weights_tensor: tensor has no scales");
      *dptr = w->arena + (n.scale ? s.s_off : s.w_off);
      if (bytes) *bytes = (size_t)(n.scale ? s.spec.scale_bytes : s.spec.weight_bytes);
      return CQ_OK;
    }
    if (n.kind == TK_LM_HEAD && !n.scale) {   // tied
      *dptr = w->embed;
      if (bytes) *bytes = (size_t)w->cfg.vocab_size * w->cfg.dim * 2;
      return CQ_OK;
    }
    return fail(CQ_EINVAL, "weights_tensor: no such tensor for this layer / config");
  }
  return fail(CQ_EINVAL, std::string("weights_tensor: unknown name ") + name);
}

extern "C" int cq_weights_wo_rows(cq_weights* w, int32_t layer, void** W, void** S) {
  if (!w || !W) return fail(CQ_EINVAL, "weights_wo_rows: null argument");
  const cq_config& c = w->cfg;
  if (layer < 0 || layer >= c.n_layers) return fail(CQ_EINVAL, "weights_wo_rows: layer out of range");
  if (!w->wo_rows) {
    const size_t qd = (size_t)c.n_heads * c.head_dim;
    const size_t wb = c.quant_type == CQ_QUANT_INT4 ? c.dim * qd / 2 : c.quant_type == CQ_QUANT_INT8 ? c.dim * qd : c.dim * qd * 2;
    const size_t sb = c.quant_type == CQ_QUANT_FP16 ? 0 : c.dim * (qd / kGroup) * 2;
    const size_t stride = align_up(align_up(wb) + sb);
    char* p = nullptr;
    if (hipMalloc((void**)&p, stride * c.n_layers) != hipSuccess)
      return fail(CQ_ENOMEM, "weights_wo_rows: allocation failed");
    int rc = CQ_OK;
    for (int l = 0; l < c.n_layers && rc == CQ_OK; ++l)
      rc = wo_from_panels(c.quant_type, w->layers[l].wo, w->layers[l].so, c.dim, (int)qd, p + stride * l,
                          sb ? reinterpret_cast<__half*>(p + stride * l + align_up(wb)) : nullptr, nullptr);
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (rc == CQ_OK && e != hipSuccess) rc = fail(CQ_EHIP, std::string("weights_wo_rows: ") + hipGetErrorString(e));
    if (rc != CQ_OK) {
      hipFree(p);
      return rc;
    }
    w->wo_rows = p;
    w->wo_rows_stride = stride;
    w->wo_rows_wbytes = align_up(wb);
  }
  *W = w->wo_rows + w->wo_rows_stride * layer;
  if (S) *S = c.quant_type == CQ_QUANT_FP16 ? nullptr : w->wo_rows + w->wo_rows_stride * layer + w->wo_rows_wbytes;
  return CQ_OK;
}

extern "C" int cq_state_create(const cq_config* cfg, const cq_weights* w, cq_state** out) {
  return cq_state_create_kv(cfg, w, CQ_KV_FP16, out);
}

extern "C" int cq_state_create_kv(const cq_config* cfg, const cq_weights* w, int32_t kv_dtype, cq_state** out) {
  if (!cfg || !out) return fail(CQ_EINVAL, "state_create: null argument");
  if (kv_dtype != CQ_KV_FP16 && kv_dtype != CQ_KV_INT8 && kv_dtype != CQ_KV_FP8)
    return fail(CQ_EINVAL, "state_create: unknown KV cache type");
  CQ_TRY(validate_config(*cfg));
  if (w && std::memcmp(cfg, &w->cfg, offsetof(cq_config, norm_eps)) != 0)
    return fail(CQ_EINVAL, "state_create: config does not match the weights");
  std::unique_ptr<cq_state> s(new cq_state);
  s->cfg = *cfg;
  s->w = w;
  const cq_config& c = *cfg;
  const size_t d = c.dim, qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
  s->kv_dtype = kv_dtype;
  s->layer_kv_halves = (size_t)c.n_kv_heads * c.max_seq_len * c.head_dim;
  const bool kvq = kv_dtype != CQ_KV_FP16;
  const size_t kv_bytes = (size_t)c.n_layers * s->layer_kv_halves * (kvq ? 1 : 2);
  const size_t sc_bytes = kvq ? (size_t)c.n_layers * c.n_kv_heads * c.max_seq_len * 4 : 0;
  // one arena: small activations, control block, history, stamps, workspaces, K, V
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return o; };
  const size_t o_x = take(d * 2), o_xb = take(qd * 2), o_q = take(qd * 2), o_k = take(kvd * 2), o_v = take(kvd * 2),
               o_inter = take((size_t)c.intermediate_size * 2), o_logits = take((size_t)c.vocab_size * 2),
               o_ctl = take(sizeof(StepCtl)), o_hist = take((size_t)c.max_seq_len * 4),
               o_tok = take((size_t)c.max_seq_len * 4), o_stamp = take((size_t)c.vocab_size * 4),
               o_attn = take(attention_workspace_bytes(c.n_heads, c.n_kv_heads, c.head_dim)),
               o_arg = take(kArgmaxPartials * 8 + 64), o_rope = take((size_t)c.head_dim / 2 * sizeof(double)),
               o_oacc = take(d * 8), o_xh = take(d * 2);
  const size_t small = off;
  const size_t o_kc = take(kv_bytes), o_vc = take(kv_bytes), o_ks = take(sc_bytes), o_vs = take(sc_bytes);
  if (hipMalloc(&s->arena, off) != hipSuccess) return fail(CQ_ENOMEM, "state_create: device allocation failed");
  char* a = s->arena;
  s->x = (__half*)(a + o_x); s->xb = (__half*)(a + o_xb); s->q = (__half*)(a + o_q); s->k = (__half*)(a + o_k);
  s->v = (__half*)(a + o_v); s->inter = (__half*)(a + o_inter); s->logits = (__half*)(a + o_logits);
  s->ctl = (StepCtl*)(a + o_ctl); s->history = (int*)(a + o_hist); s->tokens_dev = (int*)(a + o_tok);
  s->stamp = (uint32_t*)(a + o_stamp); s->attn_ws = a + o_attn; s->argmax_ws = (unsigned long long*)(a + o_arg);
  s->kcache = (__half*)(a + o_kc); s->vcache = (__half*)(a + o_vc);
  if (sc_bytes) { s->kscale = (float*)(a + o_ks); s->vscale = (float*)(a + o_vs); }
  s->rope_inv_freq = (double*)(a + o_rope);
  s->oacc = (long long*)(a + o_oacc);   // zeroed with the rest of the small region
  s->xh = (__half*)(a + o_xh);
  int rc = CQ_OK;
  auto chk = [&](hipError_t e, const char* what) {
    if (e != hipSuccess && rc == CQ_OK) rc = fail(CQ_EHIP, std::string("state_create: ") + what + ": " + hipGetErrorString(e));
  };
  chk(hipMemset(a, 0, small), "hipMemset");
  chk(hipMemset(a + o_kc, 0, kv_bytes), "hipMemset K");   // model.cu:37-38
  chk(hipMemset(a + o_vc, 0, kv_bytes), "hipMemset V");
  if (sc_bytes) {
    chk(hipMemset(a + o_ks, 0, sc_bytes), "hipMemset K scales");
    chk(hipMemset(a + o_vs, 0, sc_bytes), "hipMemset V scales");
  }
  StepCtl init{};
  init.epoch = 1u;
  init.max_history = c.max_seq_len;
  chk(hipMemcpy(s->ctl, &init, sizeof init, hipMemcpyHostToDevice), "hipMemcpy ctl");
  std::vector<double> inv_freq(c.head_dim / 2);
  rope_inv_freq_host(c.rope_theta, c.head_dim, inv_freq.data());
  chk(hipMemcpy(s->rope_inv_freq, inv_freq.data(), inv_freq.size() * sizeof(double), hipMemcpyHostToDevice),
      "hipMemcpy rope");
  chk(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
  chk(hipHostMalloc((void**)&s->host_pinned, 64 * sizeof(int), hipHostMallocDefault), "hipHostMalloc");
  chk(hipEventCreate(&s->ev0), "hipEventCreate");
  chk(hipEventCreate(&s->ev1), "hipEventCreate");
  if (rc != CQ_OK) {
    cq_state_destroy(s.release());
    return rc;
  }
  *out = s.release();
  return CQ_OK;
}

extern "C" int cq_state_destroy(cq_state* s) {
  if (!s) return CQ_OK;
  if (s->stream) hipStreamSynchronize(s->stream);
  if (s->exec) hipGraphExecDestroy(s->exec);
  if (s->graph) hipGraphDestroy(s->graph);
  if (s->exec_run) hipGraphExecDestroy(s->exec_run);
  if (s->graph_run) hipGraphDestroy(s->graph_run);
  if (s->ev0) hipEventDestroy(s->ev0);
  if (s->ev1) hipEventDestroy(s->ev1);
  if (s->host_pinned) hipHostFree(s->host_pinned);
  if (s->pf_arena) hipFree(s->pf_arena);
  if (s->pf_tokens_host) hipHostFree(s->pf_tokens_host);
  if (s->pf_copied) hipEventDestroy(s->pf_copied);
  if (s->stream) hipStreamDestroy(s->stream);
  if (s->arena) hipFree(s->arena);
  delete s;
  return CQ_OK;
}

extern "C" int cq_forward(cq_state* s, int32_t token, int32_t pos, const int32_t* history, int32_t history_len,
                          int32_t* token_out) {
  return cq_forward_ex(s, nullptr, token, pos, history, history_len, nullptr, token_out);
}

// qwen_forward (src/model.cu:183-223): the step runs on `stream` when it is
// non-NULL, else on the state's own stream (model.cu:193); weights passed
// here are bound on first use, where the reference records its graph
// (model.cu:203-213).
extern "C" int cq_forward_ex(cq_state* s, const cq_weights* w, int32_t token, int32_t pos, const int32_t* history,
                             int32_t history_len, void* stream, int32_t* token_out) {
  if (!s) return fail(CQ_EINVAL, "forward: null state");
  CQ_TRY(check_step_args(s, token, pos, history, history_len));
  CQ_TRY(bind_weights(s, w));
  CQ_TRY(ensure_graph(s));
  hipStream_t st = stream ? static_cast<hipStream_t>(stream) : s->stream;
  CQ_TRY(set_ctl(s, token, pos, history, history_len, 0, st));
  CQ_HIP(hipGraphLaunch(s->exec, st));
  CQ_HIP(hipMemcpyAsync(s->host_pinned + 8, &s->ctl->sampled, sizeof(int), hipMemcpyDeviceToHost, st));
  CQ_HIP(hipStreamSynchronize(st));
  if (token_out) *token_out = s->host_pinned[8];
  return CQ_OK;
}

extern "C" int cq_decode(cq_state* s, int32_t token, int32_t pos0, int32_t n_steps, const int32_t* history,
                         int32_t history_len, int32_t* tokens_out) {
  if (!s) return fail(CQ_EINVAL, "decode: null state");
  CQ_TRY(check_step_args(s, token, pos0, history, history_len));
  if (n_steps <= 0 || (int64_t)pos0 + n_steps > s->cfg.max_seq_len)
    return fail(CQ_ERANGE, "decode: pos0 + n_steps exceeds max_seq_len");
  // Both graphs are recorded and instantiated on the first chained decode
  // whatever its length, so a later call never records inside the span its
  // caller times.
  CQ_TRY(ensure_graph(s));
  CQ_TRY(ensure_run_graph(s));
  CQ_TRY(set_ctl(s, token, pos0, history, history_len, 1));
  CQ_HIP(hipEventRecord(s->ev0, s->stream));
  int left = n_steps;
  for (; left >= kStepsPerRun; left -= kStepsPerRun) CQ_HIP(hipGraphLaunch(s->exec_run, s->stream));
  for (; left > 0; --left) CQ_HIP(hipGraphLaunch(s->exec, s->stream));
  CQ_HIP(hipEventRecord(s->ev1, s->stream));
  if (tokens_out)
    CQ_HIP(hipMemcpyAsync(tokens_out, s->tokens_dev, (size_t)n_steps * sizeof(int), hipMemcpyDeviceToHost, s->stream));
  CQ_HIP(hipStreamSynchronize(s->stream));
  float ms = 0.f;
  CQ_HIP(hipEventElapsedTime(&ms, s->ev0, s->ev1));
  s->last_us = (double)ms * 1000.0 / n_steps;
  return CQ_OK;
}

extern "C" int cq_state_set_attention_mode(cq_state* s, int32_t mode) {
  if (!s) return fail(CQ_EINVAL, "attention mode: null state");
  if (mode != CQ_ATTN_SPLIT && mode != CQ_ATTN_WHOLE_CONTEXT) return fail(CQ_EINVAL, "attention mode: unknown mode");
  if (mode == CQ_ATTN_WHOLE_CONTEXT && s->kv_dtype != CQ_KV_FP16)
    return fail(CQ_EINVAL, "attention mode: the whole-context launch reads the fp16 cache only");
  if (mode == s->attn_mode) return CQ_OK;
  CQ_TRY(drop_graphs(s));   // the recorded steps hold the other mode's launches
  s->attn_mode = mode;
  return CQ_OK;
}

extern "C" int cq_state_last_decode_us(cq_state* s, double* us) {
  if (!s || !us) return fail(CQ_EINVAL, "null argument");
  *us = s->last_us;
  return CQ_OK;
}

extern "C" int cq_state_logits(cq_state* s, uint16_t* host_out) {
  if (!s || !host_out) return fail(CQ_EINVAL, "state_logits: null argument");
  CQ_HIP(hipMemcpyAsync(host_out, s->logits, (size_t)s->cfg.vocab_size * 2, hipMemcpyDeviceToHost, s->stream));
  CQ_HIP(hipStreamSynchronize(s->stream));
  return CQ_OK;
}

extern "C" int cq_state_fill_kv(cq_state* s, int32_t n_pos, uint64_t seed) {
  if (!s) return fail(CQ_EINVAL, "fill_kv: null state");
  if (n_pos < 0 || n_pos > s->cfg.max_seq_len) return fail(CQ_ERANGE, "fill_kv: n_pos outside [0, max_seq_len]");
  if (n_pos == 0) return CQ_OK;
  const cq_config& c = s->cfg;
  if (s->kv_dtype != CQ_KV_FP16)
    hipLaunchKernelGGL(fill_kv8_kernel, dim3(4096), dim3(256), 0, s->stream, s->kv_dtype, reinterpret_cast<int8_t*>(s->kcache),
                       reinterpret_cast<int8_t*>(s->vcache), s->kscale, s->vscale, c.n_layers, c.n_kv_heads, n_pos,
                       c.max_seq_len, c.head_dim, seed, synth_mul(1.0));
  else
    hipLaunchKernelGGL(fill_kv_kernel, dim3(8192), dim3(256), 0, s->stream, s->kcache, s->vcache, c.n_layers,
                       c.n_kv_heads, n_pos, c.max_seq_len, c.head_dim, seed, synth_mul(1.0));
  CQ_HIP(hipGetLastError());
  CQ_HIP(hipStreamSynchronize(s->stream));
  return CQ_OK;
}

// One (layer, kv head, K or V) slab of the cache: `elems` elements (whole
// tiles covering n_pos positions) at `base`, element size 2 (fp16) or 1
// (int8 / E4M3 codes, with `scales` pointing at the slab's per-position scales).
static int kv_slab(cq_state* s, int layer, int kv_head, int kind, int n_pos, char** base, size_t* elems,
                   float** scales) {
  const cq_config& c = s->cfg;
  if (layer < 0 || layer >= c.n_layers || kv_head < 0 || kv_head >= c.n_kv_heads || (kind != 0 && kind != 1))
    return fail(CQ_EINVAL, "kv access: bad layer / head / kind");
  if (n_pos < 0 || n_pos > c.max_seq_len) return fail(CQ_ERANGE, "kv access: n_pos outside [0, max_seq_len]");
  const int tile = kind == 0 ? 16 : 32;
  const int tiles = (n_pos + tile - 1) / tile;
  const size_t es = s->kv_dtype == CQ_KV_FP16 ? 2 : 1;
  *elems = (size_t)tiles * tile * c.head_dim;
  const size_t first = (size_t)layer * s->layer_kv_halves + (size_t)kv_head * c.max_seq_len * c.head_dim;
  *base = reinterpret_cast<char*>(kind == 0 ? s->kcache : s->vcache) + first * es;
  *scales = nullptr;
  if (es == 1)
    *scales = (kind == 0 ? s->kscale : s->vscale) + ((size_t)layer * c.n_kv_heads + kv_head) * c.max_seq_len;
  return CQ_OK;
}

static size_t kv_index(int kind, int t, int d, int ms, int hd) {
  return (size_t)(kind == 0 ? kv_k_offset(0, t, d, ms, hd) : kv_v_offset(0, t, d, ms, hd));
}
static size_t kv8_index(int kind, int t, int d, int ms, int hd) {
  return (size_t)(kind == 0 ? kv8_k_offset(0, t, d, ms, hd) : kv8_v_offset(0, t, d, ms, hd));
}

extern "C" int cq_state_kv_read(cq_state* s, int32_t layer, int32_t kv_head, int32_t kind, int32_t n_pos,
                                uint16_t* host_out) {
  if (!s || !host_out) return fail(CQ_EINVAL, "kv_read: null argument");
  char* base;
  size_t elems;
  float* scales;
  CQ_TRY(kv_slab(s, layer, kv_head, kind, n_pos, &base, &elems, &scales));
  const int hd = s->cfg.head_dim, ms = s->cfg.max_seq_len;
  CQ_HIP(hipStreamSynchronize(s->stream));
  if (!scales) {
    std::vector<uint16_t> tmp(elems);
    CQ_HIP(hipMemcpy(tmp.data(), base, elems * 2, hipMemcpyDeviceToHost));
    for (int t = 0; t < n_pos; ++t)
      for (int d = 0; d < hd; ++d) host_out[(size_t)t * hd + d] = tmp[kv_index(kind, t, d, ms, hd)];
    return CQ_OK;
  }
  // quantized: the dequantized value half(q * s)
  std::vector<int8_t> tmp(elems);
  std::vector<float> sc(n_pos > 0 ? n_pos : 1);
  CQ_HIP(hipMemcpy(tmp.data(), base, elems, hipMemcpyDeviceToHost));
  if (n_pos) CQ_HIP(hipMemcpy(sc.data(), scales, (size_t)n_pos * 4, hipMemcpyDeviceToHost));
  for (int t = 0; t < n_pos; ++t)
    for (int d = 0; d < hd; ++d)
      host_out[(size_t)t * hd + d] = f2h_bits(code_value(s->kv_dtype, tmp[kv8_index(kind, t, d, ms, hd)]) * sc[t]);
  return CQ_OK;
}

extern "C" int cq_state_kv_write(cq_state* s, int32_t layer, int32_t kv_head, int32_t kind, int32_t n_pos,
                                 const uint16_t* host_in) {
  if (!s || !host_in) return fail(CQ_EINVAL, "kv_write: null argument");
  char* base;
  size_t elems;
  float* scales;
  CQ_TRY(kv_slab(s, layer, kv_head, kind, n_pos, &base, &elems, &scales));
  const int hd = s->cfg.head_dim, ms = s->cfg.max_seq_len;
  CQ_HIP(hipStreamSynchronize(s->stream));
  if (!scales) {
    std::vector<uint16_t> tmp(elems);
    CQ_HIP(hipMemcpy(tmp.data(), base, elems * 2, hipMemcpyDeviceToHost));
    for (int t = 0; t < n_pos; ++t)
      for (int d = 0; d < hd; ++d) tmp[kv_index(kind, t, d, ms, hd)] = host_in[(size_t)t * hd + d];
    CQ_HIP(hipMemcpy(base, tmp.data(), elems * 2, hipMemcpyHostToDevice));
    return CQ_OK;
  }
  // quantized: each position's row with s = max|x| / code max
  std::vector<int8_t> tmp(elems), q(hd);
  std::vector<float> sc(n_pos > 0 ? n_pos : 1);
  CQ_HIP(hipMemcpy(tmp.data(), base, elems, hipMemcpyDeviceToHost));
  for (int t = 0; t < n_pos; ++t) {
    quant_row8_host(s->kv_dtype, host_in + (size_t)t * hd, hd, q.data(), &sc[t]);
    for (int d = 0; d < hd; ++d) tmp[kv8_index(kind, t, d, ms, hd)] = q[d];
  }
  CQ_HIP(hipMemcpy(base, tmp.data(), elems, hipMemcpyHostToDevice));
  if (n_pos) CQ_HIP(hipMemcpy(scales, sc.data(), (size_t)n_pos * 4, hipMemcpyHostToDevice));
  return CQ_OK;
}

// ------------------------------------------------------------ prefill
namespace {

constexpr int kPrefillChunk = 2048;   // tokens per pass through the layers
constexpr size_t kPrefillPartBytes = 64u << 20;   // split-K partials (small chunks)

int prefill_workspace(cq_state* s) {
  if (s->pf_arena) return CQ_OK;
  const cq_config& c = s->cfg;
  const size_t C = kPrefillChunk, d = c.dim, qd = (size_t)c.n_heads * c.head_dim, I = c.intermediate_size;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return o; };
  const size_t o_x = take(C * d * 2), o_a = take(C * d * 2), o_q = take(C * qd * 2), o_ao = take(C * qd * 2),
               o_i = take(C * I * 2), o_inv = take(C * 4), o_t = take(C * 4), o_p = take(kPrefillPartBytes);
  // the three parts are committed to the state together, or not at all
  char* a = nullptr;
  int* staging = nullptr;
  hipEvent_t copied = nullptr;
  if (hipMalloc(&a, off) != hipSuccess) return fail(CQ_ENOMEM, "prefill: workspace allocation failed");
  if (hipHostMalloc((void**)&staging, C * 4, hipHostMallocDefault) != hipSuccess) {
    hipFree(a);
    return fail(CQ_ENOMEM, "prefill: pinned staging allocation failed");
  }
  const hipError_t e = hipEventCreateWithFlags(&copied, hipEventDisableTiming);
  if (e != hipSuccess) {
    hipHostFree(staging);
    hipFree(a);
    return fail(CQ_EHIP, std::string("prefill: hipEventCreate: ") + hipGetErrorString(e));
  }
  s->pf_arena = a;
  s->pf_tokens_host = staging;
  s->pf_copied = copied;
  s->pf_x = (__half*)(a + o_x); s->pf_a = (__half*)(a + o_a); s->pf_q = (__half*)(a + o_q);
  s->pf_ao = (__half*)(a + o_ao); s->pf_inter = (__half*)(a + o_i); s->pf_inv = (float*)(a + o_inv);
  s->pf_tokens = (int*)(a + o_t);
  s->pf_part = (float*)(a + o_p);
  return CQ_OK;
}

// The last prompt token's tail: its row of the last layer continues through
// the decode kernels (O-proj + residual, RMSNorm + gate/up + SwiGLU, down +
// residual, final RMSNorm + lm_head, argmax into ctl->sampled); no
// repetition penalty, as in the reference's prefill loop.
int prefill_tail(cq_state* s, int M) {
  const cq_config& c = s->cfg;
  hipStream_t st = s->stream;
  const int d = c.dim, qd = c.n_heads * c.head_dim;
  CQ_HIP(hipMemcpyAsync(s->x, s->pf_x + (size_t)(M - 1) * d, (size_t)d * 2, hipMemcpyDeviceToDevice, st));
  CQ_TRY(launch_pf_row_natural(s->pf_ao + (size_t)(M - 1) * qd, s->xb, qd, c.quant_type, st));
  GemvArgs m1, m2;
  layer_gemvs(s, c.n_layers - 1, nullptr, &m1, &m2);
  fused_mlp(s, &m1, &m2);
  OMergeArgs o = layer_omerge(s, c.n_layers - 1);
  o.direct = true;   // xb holds the token's attention output
  CQ_TRY(launch_omerge(o, st));
  CQ_TRY(launch_gemv(m1, st));
  CQ_TRY(launch_gemv(m2, st));
  GemvArgs lm = lm_head_gemv(s);
  lm.stamp = nullptr;   // no penalty history
  lm.argmax_out = s->argmax_ws;
  CQ_TRY(launch_gemv(lm, st));
  return launch_argmax_reduce(s->argmax_ws, kArgmaxPartials, nullptr, &s->ctl->sampled, nullptr, nullptr, st);
}

// tokens[0..n) at positions pos0.. through every layer, M tokens at a time;
// fills the KV cache.  The last layer's O-proj / MLP run only for the last
// token, through prefill_tail (which also produces its logits and argmax).
int prefill_batched(cq_state* s, const int32_t* tokens, int n, int pos0) {
  CQ_TRY(prefill_workspace(s));
  const cq_config& c = s->cfg;
  hipStream_t st = s->stream;
  const int d = c.dim, qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim, I = c.intermediate_size;
  for (int c0 = 0; c0 < n; c0 += kPrefillChunk) {
    const int M = std::min(kPrefillChunk, n - c0);
    // the pinned staging buffer is refilled only once its previous upload is done
    CQ_HIP(hipEventSynchronize(s->pf_copied));
    std::memcpy(s->pf_tokens_host, tokens + c0, (size_t)M * 4);
    CQ_HIP(hipMemcpyAsync(s->pf_tokens, s->pf_tokens_host, (size_t)M * 4, hipMemcpyHostToDevice, st));
    CQ_HIP(hipEventRecord(s->pf_copied, st));
    CQ_TRY(launch_pf_embed(s->w->embed, s->pf_tokens, M, d, s->pf_x, st));
    for (int l = 0; l < c.n_layers; ++l) {
      const LayerW& L = s->w->layers[l];
      const bool kv8 = s->kv_dtype != CQ_KV_FP16;
      _Float16* kc = kv8 ? nullptr : (_Float16*)(s->kcache + (size_t)l * s->layer_kv_halves);
      _Float16* vc = kv8 ? nullptr : (_Float16*)(s->vcache + (size_t)l * s->layer_kv_halves);
      int8_t* kc8 = kv8 ? reinterpret_cast<int8_t*>(s->kcache) + (size_t)l * s->layer_kv_halves : nullptr;
      int8_t* vc8 = kv8 ? reinterpret_cast<int8_t*>(s->vcache) + (size_t)l * s->layer_kv_halves : nullptr;
      const size_t ls = (size_t)l * c.n_kv_heads * c.max_seq_len;
      float* ksc = kv8 ? s->kscale + ls : nullptr;
      float* vsc = kv8 ? s->vscale + ls : nullptr;
      // layer l > 0: the previous layer's down GEMM left this norm in pf_a / pf_inv
      if (l == 0) CQ_TRY(launch_pf_norm(s->pf_x, L.in_norm, c.norm_eps, M, d, s->pf_a, s->pf_inv, c.quant_type, st));
      PfGemmArgs g;
      g.mode = GM_QKV; g.quant = c.quant_type; g.A = (const _Float16*)s->pf_a; g.inv = s->pf_inv;
      g.M = M; g.N = qd + 2 * kvd; g.K = d;
      g.W[0] = L.wq; g.W[1] = L.wk; g.W[2] = L.wv;
      g.S[0] = (const _Float16*)L.sq; g.S[1] = (const _Float16*)L.sk; g.S[2] = (const _Float16*)L.sv;
      g.bias[0] = (const _Float16*)L.bq; g.bias[1] = (const _Float16*)L.bk; g.bias[2] = (const _Float16*)L.bv;
      g.rows[0] = qd; g.rows[1] = kvd; g.rows[2] = kvd;
      g.out = (_Float16*)s->pf_q; g.head_dim = c.head_dim; g.pos0 = pos0 + c0; g.max_seq = c.max_seq_len;
      g.inv_freq = s->rope_inv_freq; g.kcache = kc; g.vcache = vc;
      g.kcache8 = kc8; g.vcache8 = vc8; g.kscale = ksc; g.vscale = vsc; g.kv_fmt = s->kv_dtype;
      g.part = s->pf_part; g.part_bytes = kPrefillPartBytes;
      CQ_TRY(launch_pf_gemm(g, st));
      PfAttnArgs at;
      at.q = (const _Float16*)s->pf_q; at.kcache = kc; at.vcache = vc; at.out = (_Float16*)s->pf_ao;
      at.M = M; at.pos0 = pos0 + c0; at.n_heads = c.n_heads; at.n_kv = c.n_kv_heads; at.head_dim = c.head_dim;
      at.max_seq = c.max_seq_len;
      at.kcache8 = kc8; at.vcache8 = vc8; at.kscale = ksc; at.vscale = vsc; at.kv_fmt = s->kv_dtype;
      at.int4_layout = c.quant_type == CQ_QUANT_INT4;
      CQ_TRY(launch_pf_attention(at, st));
      if (l == c.n_layers - 1) {   // only the last token's row goes on
        if (c0 + M == n) CQ_TRY(prefill_tail(s, M));
        break;
      }
      PfGemmArgs o;
      o.mode = GM_RESID; o.quant = c.quant_type; o.A = (const _Float16*)s->pf_ao; o.M = M; o.N = d; o.K = qd;
      o.W[0] = L.wo; o.S[0] = (const _Float16*)L.so; o.panels = true; o.rows[0] = d; o.out = (_Float16*)s->pf_x;
      o.part = s->pf_part; o.part_bytes = kPrefillPartBytes;
      o.norm_w = (const _Float16*)L.post_norm; o.norm_eps = c.norm_eps;
      o.norm_out = (_Float16*)s->pf_a; o.norm_inv = s->pf_inv;
      CQ_TRY(launch_pf_gemm(o, st));
      PfGemmArgs m1;
      m1.mode = GM_SWIGLU; m1.quant = c.quant_type; m1.A = (const _Float16*)s->pf_a; m1.inv = s->pf_inv;
      m1.M = M; m1.N = I; m1.K = d; m1.W[0] = L.wg; m1.W[1] = L.wu;
      m1.S[0] = (const _Float16*)L.sg; m1.S[1] = (const _Float16*)L.su; m1.rows[0] = I; m1.rows[1] = I;
      m1.out = (_Float16*)s->pf_inter;
      m1.part = s->pf_part; m1.part_bytes = kPrefillPartBytes;
      CQ_TRY(launch_pf_gemm(m1, st));
      PfGemmArgs m2;
      m2.mode = GM_RESID; m2.quant = c.quant_type; m2.A = (const _Float16*)s->pf_inter; m2.M = M; m2.N = d; m2.K = I;
      m2.W[0] = L.wd; m2.S[0] = (const _Float16*)L.sd; m2.rows[0] = d; m2.out = (_Float16*)s->pf_x;
      m2.part = s->pf_part; m2.part_bytes = kPrefillPartBytes;
      // the next layer's input norm (every layer after this one is still to run)
      m2.norm_w = (const _Float16*)s->w->layers[l + 1].in_norm; m2.norm_eps = c.norm_eps;
      m2.norm_out = (_Float16*)s->pf_a; m2.norm_inv = s->pf_inv;
      CQ_TRY(launch_pf_gemm(m2, st));
    }
  }
  return CQ_OK;
}

}  // namespace

extern "C" int cq_prefill(cq_state* s, const int32_t* tokens, int32_t n_tokens, int32_t pos0, int32_t* token_out) {
  if (!s || !tokens) return fail(CQ_EINVAL, "prefill: null argument");
  if (n_tokens <= 0) return fail(CQ_EINVAL, "prefill: no tokens");
  if (!s->w) return fail(CQ_EINVAL, "prefill: no weights bound to the state");
  if (pos0 < 0 || (int64_t)pos0 + n_tokens > s->cfg.max_seq_len) return fail(CQ_ERANGE, "prefill: positions exceed max_seq_len");
  for (int i = 0; i < n_tokens; ++i)
    if (tokens[i] < 0 || tokens[i] >= s->cfg.vocab_size) return fail(CQ_ERANGE, "prefill: token outside the vocabulary");
  CQ_TRY(ensure_graph(s));   // recorded before any prefill work is queued on the stream
  CQ_HIP(hipEventRecord(s->ev0, s->stream));
  if (n_tokens > 1) {
    // every token through the batched path; the last one's logits and
    // argmax from its tail (no penalty history, like the reference's
    // prefill loop)
    CQ_TRY(prefill_batched(s, tokens, n_tokens, pos0));
  } else {
    // a one-token prompt is a normal decode step
    CQ_TRY(set_ctl(s, tokens[0], pos0, nullptr, 0, 0));
    CQ_HIP(hipGraphLaunch(s->exec, s->stream));
  }
  CQ_HIP(hipEventRecord(s->ev1, s->stream));
  CQ_HIP(hipMemcpyAsync(s->host_pinned + 8, &s->ctl->sampled, sizeof(int), hipMemcpyDeviceToHost, s->stream));
  CQ_HIP(hipStreamSynchronize(s->stream));
  float ms = 0.f;
  CQ_HIP(hipEventElapsedTime(&ms, s->ev0, s->ev1));
  s->last_prefill_us = (double)ms * 1000.0;
  if (token_out) *token_out = s->host_pinned[8];
  return CQ_OK;
}

extern "C" int cq_state_last_prefill_us(cq_state* s, double* us) {
  if (!s || !us) return fail(CQ_EINVAL, "null argument");
  *us = s->last_prefill_us;
  return CQ_OK;
}

// ------------------------------------------------------------ profiling
extern "C" int cq_state_profile(cq_state* s, int32_t pos, int32_t iters, int32_t max_kernels, char* names,
                                double* us_per_launch, double* bytes_per_launch, int32_t* n_kernels) {
  if (s && !s->w) return fail(CQ_EINVAL, "profile: no weights bound to the state");
  if (!s || !names || !us_per_launch || !bytes_per_launch || !n_kernels || iters <= 0)
    return fail(CQ_EINVAL, "profile: bad arguments");
  if (pos < 0 || pos >= s->cfg.max_seq_len) return fail(CQ_ERANGE, "profile: pos outside [0, max_seq_len)");
  const cq_config& c = s->cfg;
  CQ_TRY(set_ctl(s, 0, pos, nullptr, 0, 0));
  CQ_HIP(hipStreamSynchronize(s->stream));
  const double d = c.dim, I = c.intermediate_size, qd = (double)c.n_heads * c.head_dim,
               kvd = (double)c.n_kv_heads * c.head_dim, V = c.vocab_size;
  auto wbytes = [&](int quant, double rows, double cols) {
    return quant == CQ_QUANT_INT4 ? rows * cols / 2 + 2 * rows * cols / 128
         : quant == CQ_QUANT_INT8 ? rows * cols + 2 * rows * cols / 128 : 2 * rows * cols;
  };
  const int qt = c.quant_type;
  const int lmq = c.lm_head_fmt == CQ_LMHEAD_INT8 ? CQ_QUANT_INT8 : CQ_QUANT_FP16;
  const double T = pos + 1;
  struct K { const char* name; double bytes; int kind; };
  // bytes: weights + scales + activations in/out (+ bias, residual)
  const K ks[] = {
      {"qkv_rope_kvstore", wbytes(qt, qd + 2 * kvd, d) + 2 * d * 2 + 2 * (qd + 2 * kvd) * 2, 0},
      // K and V: fp16, or one code byte per element plus an fp32 scale per row
      {"attention_stage1", (s->kv_dtype == CQ_KV_FP16 ? 2.0 * c.n_kv_heads * T * c.head_dim * 2
                                                      : 2.0 * c.n_kv_heads * T * (c.head_dim + 4.0)) + 2 * qd * 2, 1},
      {"merge_o_proj", wbytes(qt, d, qd) + 8 * d * (double)c.n_heads, 2},
      {"gate_up_swiglu", wbytes(qt, 2 * I, d) + 2 * d * 2 + 8 * d + 2 * I, 3},
      {"down_residual", wbytes(qt, d, I) + 2 * I + 2 * d * 2, 4},
      {"lm_head", wbytes(lmq, V, d) + 2 * d * 2 + 2 * V, 5},
      {"argmax", 8.0 * kArgmaxPartials, 6},   // the lm_head GEMV already reduced the logits to one key per wave
      // the whole-context mode's attention + O-projection (one launch; not in the default step)
      {"attn_oproj_whole_context", 2.0 * c.n_kv_heads * T * c.head_dim * 2 + 2 * qd * 2 + wbytes(qt, d, qd) + 8 * d * (double)c.n_kv_heads, 7},
  };
  // (timed only where one kv head's K and V are at most 4 MiB: beyond that it runs for milliseconds)
  const bool short_ok = s->kv_dtype == CQ_KV_FP16 && T * c.head_dim * 4 <= 4.0 * 1024 * 1024;
  const int nk = (int)(sizeof ks / sizeof ks[0]) - (short_ok ? 0 : 1);
  int n = 0;
  for (int i = 0; i < nk && n < max_kernels; ++i, ++n) {
    const K& k = ks[i];
    const bool per_layer = k.kind <= 4 || k.kind == 7;
    const int reps = per_layer ? c.n_layers : 1;
    auto run = [&]() -> int {
      for (int l = 0; l < reps; ++l) {
        GemvArgs qkv, m1, m2;
        layer_gemvs(s, l, &qkv, &m1, &m2);
        fused_mlp(s, &m1, &m2);
        switch (k.kind) {
          case 0: CQ_TRY(launch_gemv(qkv, s->stream)); break;
          case 1: CQ_TRY(launch_attention_stage1(layer_attn(s, l), s->stream)); break;
          case 2: CQ_TRY(launch_omerge(layer_omerge(s, l), s->stream)); break;
          case 3: CQ_TRY(launch_gemv(m1, s->stream)); break;
          case 4: CQ_TRY(launch_gemv(m2, s->stream)); break;
          case 5: {
            GemvArgs lm = lm_head_gemv(s);
            lm.argmax_out = s->argmax_ws;
            CQ_TRY(launch_gemv(lm, s->stream));
            break;
          }
          case 6: CQ_TRY(launch_argmax_reduce(s->argmax_ws, kArgmaxPartials, nullptr, nullptr, nullptr, nullptr, s->stream)); break;
          case 7: CQ_TRY(launch_attn_oproj(layer_attn(s, l), layer_omerge(s, l), s->stream)); break;
        }
      }
      return CQ_OK;
    };
    CQ_TRY(run());   // warm-up
    CQ_HIP(hipEventRecord(s->ev0, s->stream));
    for (int it = 0; it < iters; ++it) CQ_TRY(run());
    CQ_HIP(hipEventRecord(s->ev1, s->stream));
    CQ_HIP(hipEventSynchronize(s->ev1));
    float ms = 0.f;
    CQ_HIP(hipEventElapsedTime(&ms, s->ev0, s->ev1));
    std::snprintf(names + 32 * n, 32, "%s", k.name);
    us_per_launch[n] = (double)ms * 1000.0 / ((double)iters * reps);
    bytes_per_launch[n] = k.bytes;
  }
  // The merged O-projection adds into the accumulator and only the down
  // projection clears it: a profile that stopped before the down projection
  // ran last would leave sums behind for the next step's first layer.
  CQ_HIP(hipMemsetAsync(s->oacc, 0, (size_t)c.dim * sizeof(long long), s->stream));
  CQ_HIP(hipStreamSynchronize(s->stream));
  *n_kernels = n;
  return CQ_OK;
}
