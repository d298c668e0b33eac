/*
 * cuqwen.h -- C ABI of the MI355X (gfx950) batch-1 Qwen2.5 decode engine.
 *
 * Every entry point takes plain pointers and sizes, returns an int status
 * (CQ_OK == 0, otherwise a CQ_E* code; cq_last_error() gives the message)
 * and never exits the process.  Device pointers are HIP device addresses;
 * `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *
 * Each declaration names the reference interface it replaces
 * (talhatahir-10xe/CuQwen, paths relative to the repository root).
 */
#ifndef CUQWEN_H
#define CUQWEN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
enum {
  CQ_OK = 0,
  CQ_EINVAL = 1,     /* bad argument / unsupported shape                      */
  CQ_EIO = 2,        /* cannot open / short read / short write                */
  CQ_EFORMAT = 3,    /* bad magic, inconsistent header, quant mismatch        */
  CQ_EHIP = 4,       /* a HIP runtime call failed                             */
  CQ_ENOMEM = 5,     /* device or host allocation failed                      */
  CQ_ERANGE = 6      /* position / token / history outside the valid range    */
};
const char* cq_last_error(void);

/* ---------------------------------------------------------------- config */
/* Weight precision tags, identical to the binary header field 9
 * (export_weights.py:24-27, include/config.h:18-33). */
enum { CQ_QUANT_FP16 = 0, CQ_QUANT_INT8 = 1, CQ_QUANT_INT4 = 2 };
/* Header field 10 (export_weights.py:262): 0 = fp16 or tied, 1 = int8. */
enum { CQ_LMHEAD_FP16 = 0, CQ_LMHEAD_INT8 = 1 };
#define CQ_MAGIC 0x5157454E       /* include/config.h:53 */
#define CQ_QUANT_GROUP 128        /* include/config.h:16 */

/* Runtime counterpart of the compile-time `struct QwenConfig`
 * (include/config.h:52-127).  Field order of the first ten ints follows the
 * binary header (export_weights.py:270-275). */
typedef struct cq_config {
  int32_t vocab_size;
  int32_t dim;
  int32_t intermediate_size;
  int32_t n_layers;
  int32_t n_heads;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t max_seq_len;
  int32_t quant_type;   /* CQ_QUANT_* */
  int32_t lm_head_fmt;  /* CQ_LMHEAD_*; with fp16, tied vs untied is `tied` */
  int32_t tied;         /* 1: lm_head aliases embed_tokens (load_weights.cpp:159) */
  float norm_eps;           /* 1e-6  (config.h:124) */
  float rope_theta;         /* 1e6   (config.h:125) */
  float repetition_penalty; /* 1.1   (config.h:126) */
} cq_config;

/* Fill `out` with one of the reference presets "0.5B" "1.5B" "3B" "7B" "14B"
 * (include/config.h:55-113) at the given precision.  lm_head_fmt/tied follow
 * the exporter's rule (export_weights.py:261): tied for 0.5B/1.5B/3B, untied
 * for 7B/14B, int8 lm_head for untied quantized models. */
int cq_config_preset(const char* model, int32_t quant_type, cq_config* out);

/* ------------------------------------------------------- weight file I/O */
/* Read and validate the 256-byte header of a weight file
 * (load_weights.cpp:46-84); fills cfg (tied is decided by file size as in
 * load_weights.cpp:139-161). */
int cq_read_header(const char* path, cq_config* cfg);

/* Write a synthetic weight file in the export_weights.py byte layout
 * (export_weights.py:267-323) from the seeded generator described in
 * cq_synth_weights; quantization follows export_weights.py:123-205. */
int cq_write_synthetic_file(const char* path, const cq_config* cfg, uint64_t seed);

/* -------------------------------------------------------------- weights */
typedef struct cq_weights cq_weights;   /* opaque: QwenWeights (load_weights.h:42-54) */

/* load_weights() (include/load_weights.h:57, src/load_weights.cpp:36-165):
 * reads the binary into device memory on the current device.  If
 * `expect` is non-NULL the header must match it (dims and quant type), as
 * the reference checks against its compiled QwenConfig. */
int cq_load_weights(const char* path, const cq_config* expect, cq_config* cfg_out, cq_weights** out);

/* Generate the same synthetic weights as cq_write_synthetic_file directly
 * in device memory (no file), bit-identical to loading that file.  Used for
 * the multi-GB presets.  No counterpart in the reference (its weights come
 * only from export_weights.py). */
int cq_synth_weights(const cq_config* cfg, uint64_t seed, cq_weights** out);

/* free_weights() (include/load_weights.h:60). */
int cq_free_weights(cq_weights* w);

/* Device pointers of one tensor, for op-level tests and tools.  `name` is one
 * of: embed, final_norm, lm_head, lm_head_scale, and per layer (layer >= 0):
 * in_norm, wq, sq, bq, wk, sk, bk, wv, sv, bv, wo, so, post_norm, wg, sg, wu,
 * su, wd, sd.  *bytes receives the tensor size.  Every tensor is held in
 * the exporter's row-major layout except the O-projection: wo is stored as
 * K/128 column panels, panel p = rows 0..N-1 of columns [128p, 128p+128)
 * (row-major within the panel), and so as [K/128][N], so that the decode's
 * merged attention + O-projection streams each head's columns contiguously
 * (converted once when the weights are loaded or synthesized). */
int cq_weights_tensor(const cq_weights* w, const char* name, int32_t layer, void** dptr, size_t* bytes);

/* Layer `layer`'s O-projection in the exporter's row-major layout: *W =
 * [dim][n_heads*head_dim] weights, *S = [dim][n_heads*head_dim/128] fp16
 * scales (NULL for fp16 weights) -- the pointers the reference's
 * LayerWeights.o_proj_weight / o_proj_scale hold (include/load_weights.h:25,
 * :35; consumed by launch_gemv_add_fp16 at src/model.cu:129).  The engine
 * keeps Wo in panels (cq_weights_tensor "wo"); the first call makes a
 * row-major copy of every layer, owned by the weights and freed with them
 * (7B INT4: 185 MB). */
int cq_weights_wo_rows(cq_weights* w, int32_t layer, void** W, void** S);

/* ---------------------------------------------------------------- state */
typedef struct cq_state cq_state;       /* opaque: QwenState (include/model.cuh:9-46) */

/* malloc_qwen_state() (include/model.cuh:48, src/model.cu:5-44).  The KV
 * cache is zeroed.  The state keeps a pointer to `w`, which must outlive it.
 * `w` may be NULL, as in the reference's two-argument
 * malloc_qwen_state(config, state): the weights are then bound by the first
 * cq_forward_ex that passes them (the reference's qwen_forward takes the
 * weights on every call and records its graph on the first,
 * src/model.cu:203-213); until then every step entry point returns
 * CQ_EINVAL. */
int cq_state_create(const cq_config* cfg, const cq_weights* w, cq_state** out);
/* free_qwen_state() (include/model.cuh:49). */
int cq_state_destroy(cq_state* s);

/* KV cache element types.  The reference keeps the cache in fp16
 * (src/model.cu:37-38); an int8 cache is its roadmap item (README.md:147).
 * CQ_KV_INT8 stores each (position, kv head) row of K and of V as
 * q = clamp(rint(x / s), -127, 127) with s = max|x| / 127 in fp32 (a zero row
 * keeps s = 0), halving the bytes the attention streams.  Scores are
 * half((q . k_q) * s_k / sqrt(head_dim)), P is rounded as half(p * s_v) for
 * the PV product. */
#define CQ_KV_FP16 0
#define CQ_KV_INT8 1
/* CQ_KV_FP8 (the roadmap item's other format, "int8/fp8") stores OCP FP8
 * E4M3 codes (bias 7, no infinities, largest finite 448) instead:
 * s = max|x| / 448, q = e4m3(x / s) rounded to nearest with ties to an even
 * mantissa; scores and P as for CQ_KV_INT8 with q read as its E4M3 value.
 * Same storage as CQ_KV_INT8 (one byte per element plus the row scales). */
#define CQ_KV_FP8 2

/* malloc_qwen_state with a choice of KV cache element type (CQ_KV_*);
 * cq_state_create is cq_state_create_kv(..., CQ_KV_FP16, ...).  With a
 * quantized cache, cq_state_kv_read returns half(value(q) * s) and
 * cq_state_kv_write quantizes each position's row as above. */
int cq_state_create_kv(const cq_config* cfg, const cq_weights* w, int32_t kv_dtype, cq_state** out);

/* qwen_forward() (include/model.cuh:51-60, src/model.cu:183-223): one decode
 * step for `token` at position `pos`, repetition penalty over
 * history[0..history_len), greedy argmax; synchronous; *token_out receives
 * the sampled id.  The first call records a HIP graph of the step; later
 * calls replay it.  Errors: CQ_ERANGE for pos outside [0, max_seq_len) or a
 * token outside the vocabulary. */
int cq_forward(cq_state* s, int32_t token, int32_t pos, const int32_t* history,
               int32_t history_len, int32_t* token_out);

/* qwen_forward() with all of its arguments (include/model.cuh:51-60,
 * src/model.cu:183-223): `w` (may be NULL once weights are bound) is bound
 * to the state if it differs from the bound set -- same config required;
 * the step graph is then recorded again -- and the step runs on `stream`
 * (a hipStream_t) when it is non-NULL, else on the state's own stream, as
 * the reference's exec_stream (model.cu:193).  Synchronous on that stream. */
int cq_forward_ex(cq_state* s, const cq_weights* w, int32_t token, int32_t pos, const int32_t* history,
                  int32_t history_len, void* stream, int32_t* token_out);

/* Greedy decode of n_steps tokens with the step chained on the device: the
 * sampled id of step i is the input of step i+1 and is appended to the
 * penalty history, without a host round trip per token (the reference's
 * caller loop, src/main.cu:95-112, does this through the host).  The
 * history starts as history[0..history_len).  tokens_out[i] receives the id
 * sampled at position pos0+i.  One host synchronisation at the end. */
int cq_decode(cq_state* s, int32_t token, int32_t pos0, int32_t n_steps,
              const int32_t* history, int32_t history_len, int32_t* tokens_out);

/* Prompt processing.  The reference's prefill loop (src/main.cu:87-92) runs
 * one qwen_forward per prompt token with no penalty history; this entry
 * point gives the same result with the tokens pushed through the layers in
 * batches (matrix-core GEMMs and a causal attention kernel, up to 2048
 * tokens per pass), the last layer's O-proj / MLP and the lm_head run for the
 * last token only (a one-token prompt is a plain decode step).  Fills the
 * KV cache for positions [pos0, pos0 + n_tokens); *token_out receives the
 * greedy id after the last prompt token and cq_state_logits its logits.
 * Errors: CQ_ERANGE for positions past max_seq_len or ids outside the
 * vocabulary. */
int cq_prefill(cq_state* s, const int32_t* tokens, int32_t n_tokens, int32_t pos0, int32_t* token_out);

/* Device time (microseconds) of the last cq_prefill call. */
int cq_state_last_prefill_us(cq_state* s, double* us);

/* Copy the fp16 logits of the last step (after the repetition penalty, as the
 * reference's state.logits holds them) to host memory (vocab_size halves). */
int cq_state_logits(cq_state* s, uint16_t* host_out);

/* Fill the KV cache of every layer for positions [0, n_pos) with seeded
 * N(0,1) fp16 values (the "KV prefilled" workloads).  Value of layer l, kv
 * head h, position t, dim d for K (kind 0) / V (kind 1) equals
 * cq_synth_normal(seed, cq_kv_stream_id(l, h, kind), t*head_dim + d, 1.0). */
int cq_state_fill_kv(cq_state* s, int32_t n_pos, uint64_t seed);

/* Read / write the KV cache of one layer and kv head for positions
 * [0, n_pos) in the reference's head-major order [n_pos][head_dim] fp16
 * (src/model.cu:112-114); the device layout itself is tiled (see
 * cq_kv_*_offset). */
int cq_state_kv_read(cq_state* s, int32_t layer, int32_t kv_head, int32_t kind, int32_t n_pos, uint16_t* host_out);
int cq_state_kv_write(cq_state* s, int32_t layer, int32_t kv_head, int32_t kind, int32_t n_pos, const uint16_t* host_in);

/* Average device time (microseconds) of the last cq_decode call per step,
 * measured with HIP events on the state's stream. */
int cq_state_last_decode_us(cq_state* s, double* us_per_step);

/* How a decode step does its attention (no counterpart in the reference,
 * whose attention is always the split-K pair, src/kernels.cu:105-324).
 * CQ_ATTN_SPLIT (the default): stage 1 over partitions of the context, then
 * the merge fused into the O-projection -- two launches per layer.
 * CQ_ATTN_WHOLE_CONTEXT: one launch per layer in which block (kv head, row
 * band) attends over the whole context itself and projects its group's
 * output; fp16 KV cache only.  Measured slower than the default at every
 * shape tried (each block streams its kv head's whole K/V), so it exists to
 * make that comparison reproducible.  Changing the mode drops the recorded
 * step graphs; they are recorded again on the next step. */
#define CQ_ATTN_SPLIT 0
#define CQ_ATTN_WHOLE_CONTEXT 1
int cq_state_set_attention_mode(cq_state* s, int32_t mode);

/* ------------------------------------------- synthetic data (host side) */
/* Deterministic approximately-normal value: Irwin-Hall sum of four 16-bit
 * uniforms from splitmix64(seed, stream, index), scaled to N(0, sigma) and
 * rounded to fp16 (returned as fp16 bits).  Bit-identical on host and
 * device. */
uint16_t cq_synth_normal(uint64_t seed, uint64_t stream, uint64_t index, float sigma);
/* Uniform integer in [0, n) from the same generator. */
uint32_t cq_synth_uniform(uint64_t seed, uint64_t stream, uint64_t index, uint32_t n);
/* Stream ids used by the weight generator and the KV filler. */
uint64_t cq_tensor_stream_id(int32_t layer, int32_t kind);
uint64_t cq_kv_stream_id(int32_t layer, int32_t kv_head, int32_t kind);

/* Host quantizer (export_weights.py:123-205): w is [rows][cols] fp16 bits;
 * q_out receives int8 [rows][cols] (quant 1) or packed int4 [rows][cols/2]
 * (quant 2); s_out receives fp16 scales [rows][cols/group]. */
int cq_quantize(int32_t quant_type, const uint16_t* w, int64_t rows, int64_t cols, int32_t group,
                void* q_out, uint16_t* s_out);

/* ------------------------------------------------- device memory helpers */
int cq_device_count(int32_t* n);
int cq_malloc(void** dptr, size_t bytes);
int cq_free(void* dptr);
int cq_memcpy_h2d(void* dst, const void* src, size_t bytes);
int cq_memcpy_d2h(void* dst, const void* src, size_t bytes);
int cq_memset(void* dptr, int value, size_t bytes);
int cq_memcpy_d2d(void* dst, const void* src, size_t bytes);
int cq_synchronize(void);

/* ------------------------------------------------------------ op level */
/* The reference's launch_* family (include/kernels.cuh:19-160).  The
 * weight-only-quant GEMVs take `quant_type` at run time instead of the
 * compile-time qweight_t; `scale` is NULL for fp16 weights.  Int8 rows are
 * `cols` bytes, int4 rows `cols/2` bytes (export_weights.py:198-199), scales
 * [rows][cols/group_size] fp16; group_size is 128 (the exporter's) or 0 for
 * one scale per row.  cols must be a multiple of 128 for quantized weights
 * and of 8 for fp16.  All are asynchronous on `stream`. */

/* launch_embedding_lookup (include/kernels.cuh:19, src/kernels.cu:85-103). */
int cq_embedding_lookup(const void* embed, const int32_t* d_token, void* out, int32_t dim, void* stream);

/* launch_rmsnorm (include/kernels.cuh:132, src/kernels.cu:689-768):
 * out = half(x * rsqrt(mean(x^2) + half(eps)) * w). */
int cq_rmsnorm(const void* x, const void* w, void* out, int32_t dim, float eps, void* stream);

/* Plain GEMV y[rows] = half(W x): the BASELINE config-1 kernel (the
 * reference has no residual-free variant; its GEMVs are
 * src/kernels.cu:402-687). */
int cq_gemv(int32_t quant_type, int32_t group_size, const void* W, const void* scale, const void* x,
            void* y, int32_t rows, int32_t cols, void* stream);

/* launch_gemv_add_fp16 (include/kernels.cuh:122, src/kernels.cu:640-687):
 * x_inout[r] = half(float(x_inout[r]) + W[r] . input). */
int cq_gemv_add(int32_t quant_type, const void* W, const void* scale, const void* input, void* x_inout,
                int32_t rows, int32_t cols, void* stream);

/* launch_fused_attn_block (include/kernels.cuh:69, src/kernels.cu:402-519):
 * q/k/v = half(W x + b) for the pre-normalised x, then NeoX RoPE at *d_pos on
 * q and k.  If norm_weight is non-NULL the RMSNorm of x is fused in front
 * (the reference passes it but leaves it unused, kernels.cu:502). */
int cq_fused_attn_block(int32_t quant_type, const void* x, const void* norm_weight,
                        const void* Wq, const void* Wk, const void* Wv,
                        const void* Sq, const void* Sk, const void* Sv,
                        const void* bq, const void* bk, const void* bv,
                        void* q_out, void* k_out, void* v_out,
                        int32_t dim, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                        const int32_t* d_pos, float rope_theta, float eps, void* stream);

/* launch_fused_mlp_stage1 (include/kernels.cuh:96, src/kernels.cu:523-585):
 * out = half(silu(Wg x) * (Wu x)); RMSNorm fused in front if norm_weight. */
int cq_fused_mlp_stage1(int32_t quant_type, const void* x, const void* norm_weight,
                        const void* Wg, const void* Wu, const void* Sg, const void* Su,
                        void* out, int32_t dim, int32_t inter_dim, float eps, void* stream);

/* launch_fused_mlp_stage2 (include/kernels.cuh:110, src/kernels.cu:590-635):
 * x[r] = half(float(x[r]) + Wd[r] . inter). */
int cq_fused_mlp_stage2(int32_t quant_type, void* x, const void* Wd, const void* Sd, const void* inter,
                        int32_t dim, int32_t inter_dim, void* stream);

/* launch_compute_logits / launch_compute_logits_int8 (include/kernels.cuh:141,
 * :152, src/kernels.cu:772-871): logits = half(W x); lm_quant is
 * CQ_LMHEAD_FP16 or CQ_LMHEAD_INT8 (scale != NULL). */
int cq_compute_logits(int32_t lm_quant, const void* x, const void* W, const void* scale, void* logits,
                      int32_t vocab, int32_t dim, void* stream);

/* launch_apply_repetition_penalty (include/kernels.cuh:49, src/kernels.cu:873-905):
 * for each distinct id in d_history[0..*d_history_len): l<0 ? l*p : l/p, applied
 * once per id (the reference's duplicate ids race, and it stops at 4096 ids). */
int cq_apply_repetition_penalty(void* logits, const int32_t* d_history, const int32_t* d_history_len,
                                int32_t vocab, float penalty, void* workspace, void* stream);
size_t cq_penalty_workspace_bytes(int32_t vocab);

/* launch_argmax (include/kernels.cuh:58, src/kernels.cu:907-961): first index
 * of the maximum (ties -> lowest index, NaN above +inf). */
int cq_argmax(const void* logits, int32_t* d_token_out, int32_t vocab, void* workspace, void* stream);
size_t cq_argmax_workspace_bytes(int32_t vocab);

/* KV cache of one layer: device layout is tiled (16-key K tiles, 32-key V
 * tiles in matrix-core operand order), head-major over kv heads with
 * max_seq_len slots per head (the reference's [n_kv][max_seq][hd] order at
 * src/model.cu:112-114 up to the tiling).  Element (kv_head, t, d) of K lives
 * at half-index cq_kv_k_offset(...), of V at cq_kv_v_offset(...). */
int64_t cq_kv_k_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim);
int64_t cq_kv_v_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim);
/* Byte offsets of element (kv_head, t, d) in an int8 / E4M3 layer cache
 * (CQ_KV_INT8 / CQ_KV_FP8): the same tiles and operand order as the fp16
 * cache, with the 8-byte operand pieces of two consecutive matrix-core
 * instructions side by side, so a lane fetches both with one 16-byte load. */
int64_t cq_kv8_k_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim);
int64_t cq_kv8_v_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim);

/* apply_rope_kernel (src/kernels.cu:370-398, launched inside
 * launch_fused_attn_block, kernels.cu:513-517): NeoX rotation of the pairs
 * (i, i + head_dim/2) of every q head (n_heads x head_dim fp16) and k head
 * (n_kv_heads x head_dim) in place at position *d_pos, freq = theta^(-2i/hd).
 * The angle is reduced in double (the reference uses fp32 fast-math). */
int cq_rope(void* q, void* k, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, const int32_t* d_pos,
            float rope_theta, void* stream);

/* The engine's KV store into its MFMA-tiled cache layout (element
 * positions: cq_kv_k_offset / cq_kv_v_offset).  The reference's
 * launch_kv_cache_store over its head-major layout is
 * cq_kv_cache_store_hm below. */
int cq_kv_cache_store(const void* k, const void* v, void* layer_k_cache, void* layer_v_cache,
                      const int32_t* d_pos, int32_t n_kv_heads, int32_t max_seq_len, int32_t head_dim,
                      void* stream);

/* The engine's decode attention over its MFMA-tiled cache (the layout
 * cq_kv_cache_store and the decode step write; not the reference's):
 * attn_out[h] = softmax(q_h . K^T / sqrt(hd)) V over keys [0, *d_pos] of kv
 * head h / (n_heads/n_kv_heads).  Split-K over the sequence sized for 256
 * CUs; `workspace` must hold cq_attention_workspace_bytes().  The
 * reference's launch_gqa_attention_decode over its head-major cache is
 * cq_gqa_attention_decode_hm below. */
int cq_gqa_attention_decode(const void* q, const void* layer_k_cache, const void* layer_v_cache, void* attn_out,
                            const int32_t* d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                            int32_t max_seq_len, void* workspace, void* stream);
size_t cq_attention_workspace_bytes(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim);

/* cq_gqa_attention_decode without a workspace argument, for callers that
 * cannot allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  No counterpart in the reference.  The split-K partials live in
 * a static device array of cq_noalloc_scratch_bytes() bytes (2.75 MiB,
 * enough for every shape cq_gqa_attention_decode accepts; larger needs
 * return CQ_ERANGE), one copy per device, held until the process ends.
 * The call allocates nothing.  All calls on one device share that copy:
 * calls that overlap on one device (two streams, two threads) race. */
int cq_gqa_attention_decode_noalloc(const void* q, const void* layer_k_cache, const void* layer_v_cache,
                                    void* attn_out, const int32_t* d_pos, int32_t n_heads, int32_t n_kv_heads,
                                    int32_t head_dim, int32_t max_seq_len, void* stream);
size_t cq_noalloc_scratch_bytes(void);

/* launch_kv_cache_store (include/kernels.cuh:37-47, src/kernels.cu:326-367):
 * k / v ([n_kv_heads * head_dim] fp16) into row *d_pos of the head-major
 * layer caches [n_kv_heads][max_seq_len][head_dim] (src/model.cu:112-114). */
int cq_kv_cache_store_hm(const void* k, const void* v, void* layer_k_cache, void* layer_v_cache,
                         const int32_t* d_pos, int32_t n_kv_heads, int32_t max_seq_len, int32_t head_dim,
                         void* stream);

/* launch_gqa_attention_decode (include/kernels.cuh:21-35, src/kernels.cu:105-324)
 * with the reference's arguments: head-major layer caches
 * [n_kv_heads][max_seq_len][head_dim], keys [0, *d_pos], 64 partitions of
 * ceil(T/64) keys, partial buffers as the reference sizes them
 * (src/model.cu:40-43): partial_out n_kv_heads*16*64*head_dim floats,
 * partial_max / partial_sum n_kv_heads*16*64 floats, entry
 * (kv_head*16 + local head)*64 + partition.  head_dim 64 or 128, up to 16
 * query heads per kv head. */
int cq_gqa_attention_decode_hm(const void* q, const void* layer_k_cache, const void* layer_v_cache, void* attn_out,
                               const int32_t* d_pos, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                               int32_t max_seq_len, float* partial_out, float* partial_max, float* partial_sum,
                               void* stream);

/* The same decode attention over an int8 layer cache (see CQ_KV_INT8; no
 * counterpart in the reference): k_new / v_new ([n_kv_heads * head_dim]
 * fp16) are quantized into position *d_pos of k_cache8 / v_cache8 (tiled,
 * one byte per element, see cq_kv8_*_offset) with their scales into k_scale / v_scale
 * ([n_kv_heads][max_seq_len] fp32), then attn_out is computed over keys
 * [0, *d_pos].  `workspace` as for cq_gqa_attention_decode. */
int cq_gqa_attention_decode_kv8(const void* q, const void* k_new, const void* v_new, void* k_cache8, void* v_cache8,
                                float* k_scale, float* v_scale, void* attn_out, const int32_t* d_pos,
                                int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                void* workspace, void* stream);
/* The same over an E4M3 layer cache (see CQ_KV_FP8; no counterpart in the
 * reference): arguments as for cq_gqa_attention_decode_kv8, the caches
 * holding E4M3 codes. */
int cq_gqa_attention_decode_fp8(const void* q, const void* k_new, const void* v_new, void* k_cache8, void* v_cache8,
                                float* k_scale, float* v_scale, void* attn_out, const int32_t* d_pos,
                                int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                void* workspace, void* stream);

/* Dequantise rows of a quantized matrix to fp32 with the device unpacking
 * path of the GEMVs (q * fp16 scale): out[rows][cols].  Test hook for the
 * bit-exact unpack check; no counterpart in the reference. */
int cq_dequantize(int32_t quant_type, int32_t group_size, const void* W, const void* scale, float* out,
                  int32_t rows, int32_t cols, void* stream);

/* ---------------------------------------------------------- timing hooks */
/* Time the plain GEMV (cq_gemv) over `n_bufs` distinct weight copies, rotated
 * per launch so the weight stream is not served from the 256 MB last-level
 * cache: `iters` launches are recorded into one HIP graph and replayed
 * between HIP events; *us_per_launch = elapsed / iters.  The
 * reference's counterpart is its cudaEvent micro-profiler
 * (benchmark/kernel_profile.cu:17-28). */
int cq_time_gemv(int32_t quant_type, int32_t group_size, int32_t n_bufs, void* const* W_list,
                 void* const* S_list, const void* x, void* y, int32_t rows, int32_t cols,
                 int32_t iters, double* us_per_launch);

/* Streaming floor: a plain read of n_bytes (16-byte non-temporal loads,
 * four 256-thread blocks per CU striding over the buffer) recorded `iters`
 * times into one HIP graph rotating over the n_bufs buffers, replayed
 * between HIP events; *us_per_launch = elapsed / iters.  The time any
 * kernel that reads n_bytes meets in the decode step's graph chain.
 * n_bytes 0 times the empty launch (per-node cost).  Measurement hook; no
 * counterpart in the reference. */
int cq_time_stream(size_t n_bytes, int32_t n_bufs, void* const* bufs, int32_t iters, double* us_per_launch);

/* Cost of a grid-wide barrier inside one kernel, the alternative to a graph
 * node boundary between dependent stages: `blocks` 256-thread blocks (at
 * most one per CU) pass `rounds` barriers; kind 0: each block publishes its
 * own flag (one 128-byte line per block) and polls all of them, kind 1:
 * one device-scope atomic counter, kind 2: the flags gathered by block 0,
 * which then releases the others through one word, kind 3: kind 2 without
 * release / acquire ordering (the signalling alone, a lower bound).  *us_per_barrier = (time with `rounds`
 * barriers - time with none) / rounds, HIP events.  Every poll is bounded:
 * *timed_out = 1 if some block gave up waiting (the figure is then not
 * valid).  Measurement hook; no counterpart in the reference. */
int cq_time_grid_barrier(int32_t kind, int32_t blocks, int32_t rounds, double* us_per_barrier, int32_t* timed_out);

/* Per-kernel profile of the decode step at position `pos` (the reference's
 * benchmark/kernel_profile.cu): each kernel of the step is launched for every
 * layer in turn (so weights rotate through all layers), `iters` rounds,
 * timed with HIP events on the state's stream.  Fills up to `max_kernels`
 * entries: names (NUL-separated into `names`, 32 bytes each), average
 * microseconds per launch, and algorithmic HBM bytes per launch. */
int cq_state_profile(cq_state* s, int32_t pos, int32_t iters, int32_t max_kernels, char* names,
                     double* us_per_launch, double* bytes_per_launch, int32_t* n_kernels);

/* ------------------------------------------------------------ tokenizer */
/* Byte-level BPE tokenizer of the Qwen2.5 family (QwenTokenizer,
 * include/tokenizer.h:18-41, src/tokenizer.cpp).  Host code only; no PCRE2
 * or JSON library is needed. */
typedef struct cq_tokenizer cq_tokenizer;

/* QwenTokenizer(ranks_json_path) (src/tokenizer.cpp:44-96): reads the
 * exporter's qwen25_bpe_ranks.json (export_weights.py:328-365: "vocab"
 * {token: id}, "added_tokens" {"id": token}; other members are skipped).
 * Errors: CQ_EIO (cannot open), CQ_EFORMAT (not that JSON layout) instead of
 * the reference's exceptions. */
int cq_tokenizer_load(const char* ranks_json_path, cq_tokenizer** out);
int cq_tokenizer_free(cq_tokenizer* t);

/* QwenTokenizer::encode (src/tokenizer.cpp:170-201): special tokens split
 * the UTF-8 text first, the rest is pre-tokenized with the Qwen2 pattern and
 * merged by byte-level BPE.  Writes *n_out ids; CQ_ERANGE (with *n_out set to
 * the count needed) when `cap` is too small.  Bytes that are not valid UTF-8
 * are kept as single characters (the reference stops at them). */
int cq_tokenizer_encode(cq_tokenizer* t, const char* text, size_t len, int32_t* ids, int32_t cap,
                        int32_t* n_out);

/* QwenTokenizer::decode / decode_single (src/tokenizer.cpp:203-238): the
 * bytes of the ids' vocabulary tokens; ids not in the vocabulary -- which
 * includes added tokens such as <|im_end|> that vocab.json lacks -- decode
 * to nothing, and a vocabulary entry spelling an added token decodes to its
 * text.  *len_out = bytes needed; CQ_ERANGE when `cap` is too small. */
int cq_tokenizer_decode(cq_tokenizer* t, const int32_t* ids, int32_t n, char* buf, size_t cap, size_t* len_out);

/* Id of a vocabulary or special token (e.g. "<|im_end|>"), -1 if absent. */
int32_t cq_tokenizer_token_id(cq_tokenizer* t, const char* token);
/* Largest id + 1. */
int32_t cq_tokenizer_vocab_size(cq_tokenizer* t);

/* QwenTokenizer::apply_chat_template (src/tokenizer.cpp:98-105):
 * "<|im_start|>{role}\n{content}<|im_end|>\n" per message, then
 * "<|im_start|>assistant\n" when add_generation_prompt.  *len_out = bytes
 * needed; CQ_ERANGE when `cap` is too small. */
int cq_chat_template(const char* const* roles, const char* const* contents, int32_t n_messages,
                     int32_t add_generation_prompt, char* buf, size_t cap, size_t* len_out);

#ifdef __cplusplus
}
#endif
#endif /* CUQWEN_H */
