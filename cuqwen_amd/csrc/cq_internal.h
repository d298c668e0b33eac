// Internal (C++) launch interface between the kernels and the engine / C ABI.
#pragma once

#include "cq_common.h"

namespace cq {

enum GemvMode { GM_STORE = 0, GM_RESID = 1, GM_SWIGLU = 2, GM_QKV = 3 };

// Fields ordered so that the struct has no padding holes: the kernels read
// their arguments in a few wide scalar loads, and a dead padding word inside
// one lets the register allocator reuse its register for a later argument
// load, which then has to wait for the whole first batch.
struct GemvArgs {
  int mode = GM_STORE;
  int quant = CQ_QUANT_FP16;
  int group = kGroup;           // 128, or 0 for one scale per row
  float eps = 1e-6f;            // fused RMSNorm epsilon
  const __half* x = nullptr;    // input vector [K]
  const __half* norm_w = nullptr;  // fused RMSNorm weight (nullptr: x is used as is)
  int K = 0;                    // contraction length
  int N = 0;                    // output rows (SWIGLU: inter rows; QKV: qd + 2 kvd)
  const void* W[3] = {nullptr, nullptr, nullptr};      // QKV: q,k,v  SWIGLU: gate, up
  const __half* S[3] = {nullptr, nullptr, nullptr};    // fp16 scales (quantized only)
  const __half* bias[3] = {nullptr, nullptr, nullptr};
  __half* out[3] = {nullptr, nullptr, nullptr};        // RESID: out[0] is read and written
  // QKV / RoPE / KV store
  int n_heads = 0, n_kv = 0;
  int head_dim = 0;
  float rope_theta = 1e6f;
  const int* d_pos = nullptr;
  const double* rope_inv_freq = nullptr;   // [head_dim/2] theta^(-2i/hd); nullptr: computed on the device
  __half* kcache = nullptr;     // layer slice, tiled layout (kv_k_offset)
  __half* vcache = nullptr;
  int max_seq = 0;
  float penalty = 1.f;          // repetition penalty applied to the stored value (logits)
  const uint32_t* stamp = nullptr;
  const uint32_t* d_epoch = nullptr;
  // STORE mode: each wave writes the argmax key of the rows it stored to
  // argmax_out[wave] (at most kArgmaxPartials waves)
  unsigned long long* argmax_out = nullptr;
  // SWIGLU with the RMSNorm fused, optional: x is first replaced by
  // half(x + x_acc * 2^-32) (the residual plus the O-projection's
  // fixed-point sum), and that vector is also written to x_out
  const long long* x_acc = nullptr;
  __half* x_out = nullptr;
  // RESID, optional: residual source (nullptr: out[0]); zero[0..zero_n) is
  // cleared once every wave has finished its rows
  const __half* resid = nullptr;
  long long* zero = nullptr;
  int zero_n = 0;
};

// Validates shapes and launches; returns CQ_OK or an error code.
int launch_gemv(const GemvArgs& a, hipStream_t stream);

// RoPE inverse frequencies 1 / theta^(2i/hd), i < hd/2, in double, computed
// on the host exactly as the oracle does (std::pow).
void rope_inv_freq_host(float theta, int head_dim, double* out);
int gemv_check(const GemvArgs& a);

int launch_dequant(int quant, int group, const void* W, const __half* S, float* out, int rows, int cols,
                   hipStream_t stream);

// ---------------------------------------------------------------- attention
struct AttnArgs {
  const __half* q = nullptr;    // [n_heads * hd] (after RoPE)
  const __half* kcache = nullptr;  // layer slice
  const __half* vcache = nullptr;
  __half* out = nullptr;        // [n_heads * hd]
  const int* d_pos = nullptr;
  int n_heads = 0, n_kv = 0, head_dim = 0, max_seq = 0;
  void* workspace = nullptr;
  // quantized cache (kcache8 / vcache8 set, kcache / vcache unused): per-(position,
  // kv head) scales [n_kv][max_seq]; the step's new k / v rows arrive in fp16
  // (k_new / v_new, [n_kv * hd]) and are quantized into position *d_pos here
  int8_t* kcache8 = nullptr;
  int8_t* vcache8 = nullptr;
  float* kscale = nullptr;
  float* vscale = nullptr;
  const __half* k_new = nullptr;
  const __half* v_new = nullptr;
  int kv_fmt = CQ_KV_INT8;   // codes of kcache8 / vcache8: CQ_KV_INT8 or CQ_KV_FP8
};
size_t attention_workspace_bytes(int n_heads, int n_kv, int head_dim);
int launch_attention(const AttnArgs& a, hipStream_t stream);
int attention_max_parts(int n_kv);
// Attention stage 1 alone (the partials stay in the workspace, or the output
// in `out` when one partition covers the context).
int launch_attention_stage1(const AttnArgs& a, hipStream_t stream);

// Attention merge + O-projection split over heads (cq_omerge.hip): merges
// the stage-1 partials of each head (or takes the single-partition output
// from attn) and adds Wo * attention to acc as 64-bit fixed point (2^-32).
struct OMergeArgs {
  const void* workspace = nullptr;   // stage-1 partials (attention workspace layout)
  const __half* attn = nullptr;      // stage 1's output when it used one partition
  const void* W = nullptr;           // Wo [N][K]
  const __half* S = nullptr;         // its group-128 scales (quantized)
  long long* acc = nullptr;          // [N], added to
  const int* d_pos = nullptr;
  int quant = CQ_QUANT_FP16;
  int n_heads = 0, n_kv = 0, head_dim = 0;
  int K = 0, N = 0;                  // K = n_heads * head_dim
  int Pmax = 0;                      // partition slots per kv head (stage 1's grid)
  int bands = 0;                     // set by the launcher
  bool direct = false;               // attn holds the finished output (no partials)
};
int launch_omerge(const OMergeArgs& a, hipStream_t stream);
// Converts a row-major [N][K] O-projection (and its [N][K/128] scales) in
// place into K/128 column panels [N][128] (scales [K/128][N]), the layout
// launch_omerge and the prefill O-projection read; tmp holds N*K weight bytes.
int wo_to_panels(int quant, void* W, __half* S, int N, int K, void* tmp, hipStream_t stream);
int wo_from_panels(int quant, const void* W, const __half* S, int N, int K, void* W_rows, __half* S_rows,
                   hipStream_t stream);
int omerge_plan(int quant, int head_dim, int n_heads, int N, int* hpb, int* bands, int* rounds, int* wm);
// Short contexts (cq_omerge.hip): attention over the whole fp16 cache and
// the O-projection in one launch, block (kv head, row band) recomputing its
// group's attention; same accumulator as launch_omerge.
int launch_attn_oproj(const AttnArgs& at, const OMergeArgs& a, hipStream_t stream);
int attn_oproj_plan(int quant, int head_dim, int n_heads, int n_kv, int N, int* bands, int* rounds, int* cpl);
// Head-major cache path (cq_attention_hm.hip): the reference's layout and
// partial buffers (partial index (kv_head * 16 + head) * 64 + partition).
int launch_attention_hm(const __half* q, const __half* kc, const __half* vc, __half* out, const int* d_pos,
                        int n_heads, int n_kv, int head_dim, int max_seq, float* part_out, float* part_max,
                        float* part_sum, hipStream_t stream);
int launch_kv_store_hm(const __half* k, const __half* v, __half* kc, __half* vc, const int* d_pos, int n_kv,
                       int max_seq, int hd, hipStream_t stream);

// ---------------------------------------------------------------- prefill
// M-token GEMM on the matrix cores (cq_prefill.hip).  A: [M][K] activations
// in the layout of the weights' format (int4: permuted 8-groups, odd
// elements / 16; int8 / fp16: natural); rows[]: rows of W[0..2] (QKV: q, k, v;
// otherwise rows[0] = N); out: RESID -> [M][N] residual (natural, in place),
// SWIGLU -> [M][N] (permuted), QKV -> q [M][rows[0]] (natural) + KV cache.
struct PfGemmArgs {
  int mode = GM_RESID;
  int quant = CQ_QUANT_FP16;
  const _Float16* A = nullptr;
  const float* inv = nullptr;   // [M] RMSNorm scale (QKV, SWIGLU)
  int M = 0, N = 0, K = 0;
  const void* W[3] = {nullptr, nullptr, nullptr};
  const _Float16* S[3] = {nullptr, nullptr, nullptr};
  const _Float16* bias[3] = {nullptr, nullptr, nullptr};
  int rows[3] = {0, 0, 0};
  _Float16* out = nullptr;
  int head_dim = 0, pos0 = 0, max_seq = 0;
  const double* inv_freq = nullptr;
  _Float16* kcache = nullptr;
  _Float16* vcache = nullptr;
  // split-K workspace (fp32 partials); nullptr: no split
  float* part = nullptr;
  size_t part_bytes = 0;
  // quantized cache (instead of kcache / vcache): rows quantized per (token, kv head)
  int8_t* kcache8 = nullptr;
  int8_t* vcache8 = nullptr;
  float* kscale = nullptr;   // [n_kv][max_seq] of this layer
  float* vscale = nullptr;
  int kv_fmt = CQ_KV_INT8;   // CQ_KV_INT8 / CQ_KV_FP8 codes
  bool panels = false;       // W[0] / S[0] in 128-column panels (wo_to_panels), not row-major
  // RESID only, optional: RMSNorm of the updated rows (as launch_pf_norm) into
  // norm_out / norm_inv with weight norm_w
  const _Float16* norm_w = nullptr;
  float norm_eps = 0.f;
  _Float16* norm_out = nullptr;
  float* norm_inv = nullptr;
};
struct PfAttnArgs {
  const _Float16* q = nullptr;   // [M][n_heads * hd] natural
  const _Float16* kcache = nullptr;
  const _Float16* vcache = nullptr;
  _Float16* out = nullptr;       // [M][n_heads * hd] permuted
  int M = 0, pos0 = 0, n_heads = 0, n_kv = 0, head_dim = 0, max_seq = 0;
  const int8_t* kcache8 = nullptr;   // quantized cache (kv_fmt codes) instead of kcache / vcache
  const int8_t* vcache8 = nullptr;
  const float* kscale = nullptr;
  const float* vscale = nullptr;
  int kv_fmt = CQ_KV_INT8;
  bool int4_layout = false;   // out in the int4 GEMM input layout (else natural order)
};
int launch_pf_norm(const __half* x, const __half* w, float eps, int M, int dim, __half* A, float* inv, int quant,
                   hipStream_t stream);
int launch_pf_embed(const __half* embed, const int* tokens, int M, int dim, __half* x, hipStream_t stream);
int launch_pf_row_natural(const __half* src, __half* dst, int n, int quant, hipStream_t stream);
int launch_pf_gemm(const PfGemmArgs& a, hipStream_t stream);
int launch_pf_attention(const PfAttnArgs& a, hipStream_t stream);

// --------------------------------------------------------------- misc ops
int launch_embedding(const __half* embed, const int* d_token, __half* out, int dim, hipStream_t stream);
int launch_rmsnorm(const __half* x, const __half* w, __half* out, int dim, float eps, hipStream_t stream);
int launch_rope(__half* q, __half* k, int n_heads, int n_kv, int head_dim, const int* d_pos, float theta,
                hipStream_t stream);
int launch_kv_store(const __half* k, const __half* v, __half* kc, __half* vc, const int* d_pos, int n_kv,
                    int max_seq, int hd, hipStream_t stream);
// Marks ids d_history[0..*d_history_len) in `stamp` with the value *d_epoch.
int launch_stamp_history(uint32_t* stamp, const int* d_history, const int* d_history_len, int vocab,
                         const uint32_t* d_epoch, hipStream_t stream);
// Penalty on logits for stamped ids (stand-alone form of the lm_head epilogue).
int launch_penalty_apply(__half* logits, const uint32_t* stamp, const uint32_t* d_epoch, int vocab,
                         float penalty, hipStream_t stream);

// Decode-step control block in device memory.
struct StepCtl {
  // written by the host before a step / a chained decode (all 8 words)
  int token;        // input token of the next step
  int pos;          // position of the next step
  int history_len;  // ids in the history buffer
  int chain;        // 1: the argmax feeds the next step (token, pos+1, history append)
  int step;         // index into tokens_out for chained decode
  // maintained on the device
  int sampled;      // id sampled by the last step
  int max_history;  // history buffer capacity
  uint32_t epoch;   // penalty stamp epoch, set by the host with each new history
};

// Argmax over fp16 logits (ties -> lowest index).  `partials` holds
// kArgmaxBlocks uint64 keys; `ctl` (optional) receives the token and, when
// ctl->chain, advances the step; `tokens_out` (optional) records the token at
// ctl->step.
constexpr int kArgmaxBlocks = 256;
constexpr int kArgmaxPartials = 4096;   // keys written by the lm_head GEMV (one per wave)
// Work of the next chained step's prologue folded into the argmax reduce:
// when ctl->chain, the sampled id's embedding row goes to x and its penalty
// stamp gets the current epoch.  All null: no prologue work.
struct StepBegin {
  const __half* embed = nullptr;
  __half* x = nullptr;
  int dim = 0;
  uint32_t* stamp = nullptr;
};
// Reduces n argmax keys and does the step bookkeeping of launch_argmax.
int launch_argmax_reduce(const unsigned long long* partials, int n, StepCtl* ctl, int* d_token_out, int* history,
                         int* tokens_out, hipStream_t stream, StepBegin next = StepBegin());
int launch_argmax(const __half* logits, int vocab, unsigned long long* partials, StepCtl* ctl,
                  int* d_token_out, int* history, int* tokens_out, hipStream_t stream);

// Step prologue: embedding of ctl->token into x, stamp the history with a new
// epoch.
int launch_step_begin(const __half* embed, StepCtl* ctl, const int* history, uint32_t* stamp, __half* x,
                      int dim, int vocab, hipStream_t stream);

}  // namespace cq
