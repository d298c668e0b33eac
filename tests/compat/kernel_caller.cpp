// The reference's op-level caller, benchmark/kernel_profile.cu:66-85, written
// against include/cuqwen_compat.hpp: the same buffers (sized from QwenConfig
// and WEIGHT_ROW_STRIDE / QUANT_GROUP_SIZE / PARTIAL_HEAD_SLOTS /
// ATTN_PARTITIONS) and the same launch_* calls in the same order, with seeded
// data in place of its zeroed buffers so the results can be checked: every
// input and every op's output is written to <outdir> for
// tests/test_gpu_compat_ops.py to compare with the oracle.
//
//   ops <outdir> <pos>
//       the kernel_profile sequence at context position <pos>, plus
//       launch_compute_logits_int8 (include/kernels.cuh:152)
//   oproj <bin> <outdir> <layer>
//       load_weights, then launch_gemv_add_fp16 on the loaded
//       LayerWeights.o_proj_weight / o_proj_scale of <layer> the way
//       src/model.cu:129 uses them
//
// Built by cuqwen_amd/build.py once per precision (-DQUANT_INT8, -DQUANT_INT4,
// fp16) for the 0.5B and 1.5B presets.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "cuqwen_compat.hpp"

#define HIP_OK(call)                                                                              \
  do {                                                                                            \
    hipError_t e_ = (call);                                                                       \
    if (e_ != hipSuccess) {                                                                       \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(1);                                                                               \
    }                                                                                             \
  } while (0)

static std::string g_dir;

struct Rng {   // xorshift64*, seeded per buffer
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
  uint64_t next() {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1Dull;
  }
  float uniform() { return (float)((next() >> 40) * (1.0 / 16777216.0)); }   // [0, 1)
  float normal() {   // sum of four uniforms, standardised
    float a = 0.f;
    for (int i = 0; i < 4; ++i) a += uniform();
    return (a - 2.f) * 1.7320508f;
  }
};

static void dump(const char* name, const void* host, size_t bytes) {
  const std::string path = g_dir + "/" + name + ".bin";
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(host, 1, bytes, f) != bytes) {
    std::fprintf(stderr, "cannot write %s\n", path.c_str());
    std::exit(1);
  }
  std::fclose(f);
}

static void dump_dev(const char* name, const void* dev, size_t bytes) {
  std::vector<char> h(bytes);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(h.data(), dev, bytes, hipMemcpyDeviceToHost));
  dump(name, h.data(), bytes);
}

template <typename T>
static T* dmalloc(size_t n) {
  T* p = nullptr;
  HIP_OK(hipMalloc(&p, n * sizeof(T)));
  HIP_OK(hipMemset(p, 0, n * sizeof(T)));
  return p;
}

// A device buffer of `n` fp16 values sigma * N(0,1) (+ mean), also dumped.
static __half* dhalf(const char* name, size_t n, uint64_t seed, float sigma, float mean = 0.f) {
  std::vector<__half> h(n);
  Rng r(seed);
  for (auto& v : h) v = __float2half(mean + sigma * r.normal());
  __half* d = dmalloc<__half>(n);
  HIP_OK(hipMemcpy(d, h.data(), n * 2, hipMemcpyHostToDevice));
  dump(name, h.data(), n * 2);
  return d;
}

// Weights of this build's precision, [rows][cols] in the exporter's layout:
// int8 / int4 bytes drawn uniformly over every code, fp16 N(0, 0.02).
static qweight_t* dweight(const char* name, size_t rows, size_t cols, uint64_t seed) {
#ifdef QUANT_ENABLED
  const size_t n = rows * WEIGHT_ROW_STRIDE(cols);
  std::vector<uint8_t> h(n);
  Rng r(seed);
  for (auto& b : h) {
    b = (uint8_t)(r.next() >> 56);
#ifdef QUANT_INT8
    if (b == 0x80) b = 0x81;   // the exporter emits [-127, 127]
#endif
  }
  qweight_t* d = dmalloc<qweight_t>(n);
  HIP_OK(hipMemcpy(d, h.data(), n, hipMemcpyHostToDevice));
  dump(name, h.data(), n);
  return d;
#else
  return reinterpret_cast<qweight_t*>(dhalf(name, rows * cols, seed, 0.02f));
#endif
}

// Scales [rows][cols / QUANT_GROUP_SIZE], positive, sized so that outputs are
// O(1); nullptr for fp16 builds (the reference passes nullptr there too).
static __half* dscale(const char* name, size_t rows, size_t cols, uint64_t seed) {
#ifdef QUANT_ENABLED
#ifdef QUANT_INT8
  const float base = 0.02f / 127.f * 2.6f;
#else
  const float base = 0.02f / 7.f * 2.6f;
#endif
  const size_t n = rows * (cols / QUANT_GROUP_SIZE);
  std::vector<__half> h(n);
  Rng r(seed);
  for (auto& v : h) v = __float2half(base * (0.5f + r.uniform()));
  __half* d = dmalloc<__half>(n);
  HIP_OK(hipMemcpy(d, h.data(), n * 2, hipMemcpyHostToDevice));
  dump(name, h.data(), n * 2);
  return d;
#else
  (void)name; (void)rows; (void)cols; (void)seed;
  return nullptr;
#endif
}

static int ops(int pos) {
  QwenConfig cfg;
  const int dim = cfg.dim, inter = cfg.intermediate_size, head_dim = cfg.head_dim;
  const int n_heads = cfg.n_heads, n_kv = cfg.n_kv_heads;
  const int q_dim = n_heads * head_dim, kv_dim = n_kv * head_dim;
  const int msl = cfg.max_seq_len, vocab = cfg.vocab_size;
  if (pos < 0 || pos >= msl) return 2;

  // buffers, as kernel_profile.cu:38-62 allocates them
  __half* x = dhalf("x0", dim, 1, 1.f);
  __half* xb = dmalloc<__half>(dim);
  __half* att = dmalloc<__half>(dim);
  __half *q = dmalloc<__half>(q_dim), *k = dmalloc<__half>(kv_dim), *v = dmalloc<__half>(kv_dim);
  __half* gate = dmalloc<__half>(inter);
  __half* logits = dmalloc<__half>(vocab);
  __half* norm_w = dhalf("norm_w", dim, 2, 0.1f, 1.f);
  int* d_pos = dmalloc<int>(1);
  HIP_OK(hipMemcpy(d_pos, &pos, sizeof(int), hipMemcpyHostToDevice));
  int *d_tok = dmalloc<int>(1), *d_samp = dmalloc<int>(1), *d_hist = dmalloc<int>(msl), *d_hlen = dmalloc<int>(1);
  const int tok = 12345 % vocab, hlen = 500;
  std::vector<int> hist(hlen);
  {
    Rng r(3);
    for (int i = 0; i < hlen; ++i) hist[i] = (int)(r.next() % 4096);   // duplicates included
  }
  HIP_OK(hipMemcpy(d_tok, &tok, sizeof(int), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_hist, hist.data(), hlen * sizeof(int), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_hlen, &hlen, sizeof(int), hipMemcpyHostToDevice));
  dump("hist", hist.data(), hlen * sizeof(int));

  qweight_t* Wq = dweight("Wq", q_dim, dim, 10);
  qweight_t* Wk = dweight("Wk", kv_dim, dim, 11);
  qweight_t* Wv = dweight("Wv", kv_dim, dim, 12);
  qweight_t* Wo = dweight("Wo", dim, q_dim, 13);
  qweight_t* Wg = dweight("Wg", inter, dim, 14);
  qweight_t* Wu = dweight("Wu", inter, dim, 15);
  qweight_t* Wd = dweight("Wd", dim, inter, 16);
  __half* Sq = dscale("Sq", q_dim, dim, 20);
  __half* Sk = dscale("Sk", kv_dim, dim, 21);
  __half* Sv = dscale("Sv", kv_dim, dim, 22);
  __half* So = dscale("So", dim, q_dim, 23);
  __half* Sg = dscale("Sg", inter, dim, 24);
  __half* Su = dscale("Su", inter, dim, 25);
  __half* Sd = dscale("Sd", dim, inter, 26);
  __half* bq = dhalf("bq", q_dim, 30, 0.02f);
  __half* bk = dhalf("bk", kv_dim, 31, 0.02f);
  __half* bv = dhalf("bv", kv_dim, 32, 0.02f);
  // embedding and fp16 lm_head tables; only the looked-up row of the
  // embedding is dumped
  __half* embed = dmalloc<__half>((size_t)vocab * dim);
  {
    std::vector<__half> h((size_t)vocab * dim);
    Rng r(40);
    for (auto& e : h) e = __float2half(0.5f * r.normal());
    HIP_OK(hipMemcpy(embed, h.data(), h.size() * 2, hipMemcpyHostToDevice));
    dump("embed_row", h.data() + (size_t)tok * dim, (size_t)dim * 2);
  }
  __half* lmhead = dhalf("lmhead", (size_t)vocab * dim, 41, 0.02f);
  int8_t* lmq = dmalloc<int8_t>((size_t)vocab * dim);
  {
    std::vector<int8_t> h((size_t)vocab * dim);
    Rng r(42);
    for (auto& b : h) b = (int8_t)((int)(r.next() % 255) - 127);
    HIP_OK(hipMemcpy(lmq, h.data(), h.size(), hipMemcpyHostToDevice));
    dump("lmq", h.data(), h.size());
  }
  __half* lms = nullptr;
  {
    const size_t n = (size_t)vocab * (dim / QUANT_GROUP_SIZE);
    std::vector<__half> h(n);
    Rng r(43);
    for (auto& e : h) e = __float2half(4e-4f * (0.5f + r.uniform()));
    lms = dmalloc<__half>(n);
    HIP_OK(hipMemcpy(lms, h.data(), n * 2, hipMemcpyHostToDevice));
    dump("lms", h.data(), n * 2);
  }
  // KV cache for one layer, head-major [n_kv][msl][head_dim]; positions
  // before pos hold N(0,1) values (kernel_profile leaves them zero)
  __half *kc = dmalloc<__half>((size_t)n_kv * msl * head_dim), *vc = dmalloc<__half>((size_t)n_kv * msl * head_dim);
  {
    std::vector<__half> hk((size_t)n_kv * pos * head_dim), hv(hk.size());
    Rng rk(50), rv(51);
    for (auto& e : hk) e = __float2half(rk.normal());
    for (auto& e : hv) e = __float2half(rv.normal());
    for (int h = 0; h < n_kv; ++h) {
      HIP_OK(hipMemcpy(kc + (size_t)h * msl * head_dim, hk.data() + (size_t)h * pos * head_dim,
                       (size_t)pos * head_dim * 2, hipMemcpyHostToDevice));
      HIP_OK(hipMemcpy(vc + (size_t)h * msl * head_dim, hv.data() + (size_t)h * pos * head_dim,
                       (size_t)pos * head_dim * 2, hipMemcpyHostToDevice));
    }
    dump("kc_prefix", hk.data(), hk.size() * 2);
    dump("vc_prefix", hv.data(), hv.size() * 2);
  }
  size_t splits = (size_t)n_kv * PARTIAL_HEAD_SLOTS * ATTN_PARTITIONS;
  float *po = dmalloc<float>(splits * head_dim), *pmx = dmalloc<float>(splits), *psm = dmalloc<float>(splits);

  __half eps = __float2half(cfg.norm_eps);
  hipStream_t s = 0;
  // kernel_profile.cu:66-85, in order; each op's output dumped after it
  launch_rmsnorm(x, norm_w, att, dim, eps, s);
  dump_dev("01_att", att, dim * 2);
  launch_fused_attn_block(att, norm_w, Wq, Wk, Wv, Sq, Sk, Sv, bq, bk, bv, q, k, v, dim, q_dim, kv_dim, n_heads, n_kv,
                          head_dim, d_pos, cfg.rope_theta, eps, s);
  dump_dev("02_q", q, q_dim * 2);
  dump_dev("02_k", k, kv_dim * 2);
  dump_dev("02_v", v, kv_dim * 2);
  launch_kv_cache_store(k, v, kc, vc, d_pos, n_kv, msl, head_dim, s);
  {
    // rows pos-1 .. pos+1 of every kv head: the new row and both neighbours
    std::vector<__half> rows;
    for (__half* c : {kc, vc})
      for (int h = 0; h < n_kv; ++h) {
        const int lo = pos > 0 ? pos - 1 : 0, hi = pos + 1 < msl ? pos + 1 : pos;
        std::vector<__half> r((size_t)(hi - lo + 1) * head_dim);
        HIP_OK(hipDeviceSynchronize());
        HIP_OK(hipMemcpy(r.data(), c + ((size_t)h * msl + lo) * head_dim, r.size() * 2, hipMemcpyDeviceToHost));
        rows.insert(rows.end(), r.begin(), r.end());
      }
    dump("03_kv_rows", rows.data(), rows.size() * 2);
  }
  launch_gqa_attention_decode(q, kc, vc, xb, d_pos, n_heads, n_kv, head_dim, msl, po, pmx, psm, s);
  dump_dev("04_xb", xb, q_dim * 2);
  launch_gemv_add_fp16(Wo, So, xb, x, dim, q_dim, s);
  dump_dev("05_x", x, dim * 2);
  launch_fused_mlp_stage1(att, norm_w, Wg, Wu, Sg, Su, gate, dim, inter, eps, s);
  dump_dev("06_gate", gate, inter * 2);
  launch_fused_mlp_stage2(x, Wd, Sd, gate, dim, inter, s);
  dump_dev("07_x", x, dim * 2);
  launch_embedding_lookup(embed, d_tok, x, dim, s);
  dump_dev("08_x", x, dim * 2);
  launch_rmsnorm(x, norm_w, xb, dim, eps, s);
  dump_dev("09_xb", xb, dim * 2);
  launch_compute_logits(xb, lmhead, logits, vocab, dim, s);
  dump_dev("10_logits", logits, (size_t)vocab * 2);
  launch_apply_repetition_penalty(logits, d_hist, d_hlen, vocab, __float2half(1.1f), s);
  dump_dev("11_logits", logits, (size_t)vocab * 2);
  launch_argmax(logits, d_samp, vocab, s);
  dump_dev("12_samp", d_samp, sizeof(int));
  launch_compute_logits_int8(xb, lmq, lms, logits, vocab, dim, s);
  dump_dev("13_logits", logits, (size_t)vocab * 2);
  launch_argmax(logits, d_samp, vocab, s);   // a second call reuses the wrapper's workspace
  dump_dev("14_samp", d_samp, sizeof(int));
  HIP_OK(hipDeviceSynchronize());

  for (void* p : std::initializer_list<void*>{x, xb, att, q, k, v, gate, logits, norm_w, d_pos, d_tok, d_samp, d_hist,
                                               d_hlen, Wq, Wk, Wv, Wo, Wg, Wu, Wd, bq, bk, bv, embed, lmhead, lmq, lms,
                                               kc, vc, po, pmx, psm})
    HIP_OK(hipFree(p));
  for (void* p : std::initializer_list<void*>{Sq, Sk, Sv, So, Sg, Su, Sd})
    if (p) HIP_OK(hipFree(p));
  std::printf("{\"ok\": true, \"pos\": %d, \"tok\": %d}\n", pos, tok);
  return 0;
}

static int oproj(const std::string& bin, int layer) {
  QwenWeights weights;
  QwenConfig config = load_weights(bin, weights);
  if (layer < 0 || layer >= config.n_layers) return 2;
  const int dim = config.dim, q_dim = config.n_heads * config.head_dim;
  __half* xb = dhalf("xb", q_dim, 60, 1.f);
  __half* x = dhalf("x0", dim, 61, 1.f);
  const LayerWeights& L = weights.layers[layer];
  launch_gemv_add_fp16(L.o_proj_weight, L.o_proj_scale, xb, x, dim, q_dim, 0);
  dump_dev("x1", x, dim * 2);
  HIP_OK(hipFree(xb));
  HIP_OK(hipFree(x));
  free_weights(weights, config);
  std::printf("{\"ok\": true, \"layer\": %d}\n", layer);
  return 0;
}

int main(int argc, char** argv) {
  try {
    if (argc == 4 && std::strcmp(argv[1], "ops") == 0) {
      g_dir = argv[2];
      return ops(std::atoi(argv[3]));
    }
    if (argc == 5 && std::strcmp(argv[1], "oproj") == 0) {
      g_dir = argv[3];
      return oproj(argv[2], std::atoi(argv[4]));
    }
  } catch (const std::exception& e) {
    std::fprintf(stderr, "kernel_caller: %s\n", e.what());
    return 1;
  }
  std::fprintf(stderr, "usage: kernel_caller ops <outdir> <pos>\n       kernel_caller oproj <bin> <outdir> <layer>\n");
  return 2;
}
