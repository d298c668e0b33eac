// Host-code sanitizer driver: oracle/oracle.cpp, cuqwen_amd/csrc/cq_format.cpp
// and cuqwen_amd/csrc/cq_tokenizer.cpp built with -fsanitize=address,undefined
// (tests/sanitize/Makefile) and driven through their C entry points with
// valid and malformed inputs: quantizer, GEMV, norm, RoPE, attention (fp16,
// int8, E4M3), argmax, penalty, tiny-model decode in every precision and
// lm_head form, weight-file write / read / truncated / bad magic, presets,
// tokenizer load / encode / decode / chat template on random and invalid
// UTF-8 and on malformed ranks files.  Any sanitizer report aborts the
// process with a non-zero status; success prints "sanitize ok".
// Test infrastructure only (run by tests/test_sanitizers.py, CPU).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "cuqwen.h"

extern "C" {
void or_quantize(int quant, const uint16_t* w, int64_t rows, int64_t cols, int64_t group, uint8_t* q, uint16_t* s);
void or_gemv(int quant, const uint8_t* W, const uint16_t* S, const uint16_t* x, float* y, int64_t rows, int64_t cols,
             int64_t group, int mode);
void or_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int64_t dim, float eps, int mode);
void or_rope(uint16_t* v, int n_heads, int hd, int pos, float theta);
void or_attention(const uint16_t* q, const uint16_t* K, const uint16_t* V, uint16_t* out, int n_heads, int n_kv,
                  int hd, int64_t stride, int T, int mode, int nparts);
void or_attention_kvq(const uint16_t* q, const int8_t* Kq, const float* Ks, const int8_t* Vq, const float* Vs,
                      uint16_t* out, int n_heads, int n_kv, int hd, int64_t stride, int T, int mode, int nparts,
                      int fmt);
void or_quant_row_i8(const uint16_t* x, int n, int8_t* q, float* s);
void or_quant_row_f8(const uint16_t* x, int n, uint8_t* q, float* s);
void or_e4m3_encode(const float* x, int64_t n, uint8_t* out);
void or_e4m3_decode(const uint8_t* b, int64_t n, float* out);
int or_argmax(const uint16_t* logits, int vocab);
void or_penalty(uint16_t* logits, const int* hist, int n, int vocab, float pen);
uint16_t or_f2h(float f);
void* or_model_synth(const int* cfg11, uint64_t seed, int kv_slots);
void* or_model_load(const char* path, int kv_slots);
void or_model_free(void* h);
void or_model_set_nparts(void* h, int nparts);
void or_model_set_kv8(void* h, int on);
void or_model_fill_kv(void* h, int n_pos, uint64_t seed);
int or_model_forward(void* h, int token, int pos, const int* hist, int hlen, int mode);
void or_model_logits(void* h, uint16_t* out);
int64_t or_model_tensor(void* h, int layer, int kind, int which, void* out);
}

static int g_fail = 0;
#define CHECK(c)                                                         \
  do {                                                                   \
    if (!(c)) {                                                          \
      std::fprintf(stderr, "check failed: %s (%s:%d)\n", #c, __FILE__, __LINE__); \
      ++g_fail;                                                          \
    }                                                                    \
  } while (0)

static std::mt19937_64 rng(12345);
static std::vector<uint16_t> halves(size_t n, float sd) {
  std::normal_distribution<float> nd(0.f, sd);
  std::vector<uint16_t> v(n);
  for (auto& h : v) h = or_f2h(nd(rng));
  return v;
}

static void oracle_ops() {
  const int rows = 24, cols = 384;
  auto w = halves((size_t)rows * cols, 0.02f);
  auto x = halves(cols, 1.f);
  for (int quant = 0; quant <= 2; ++quant)
    for (int group : {128, 0}) {
      std::vector<uint8_t> q((size_t)rows * cols * 2);
      std::vector<uint16_t> s((size_t)rows * (cols / 128) + 1);
      const uint8_t* W = reinterpret_cast<const uint8_t*>(w.data());
      if (quant) {
        or_quantize(quant, w.data(), rows, cols, group, q.data(), s.data());
        W = q.data();
      }
      std::vector<float> y(rows);
      for (int mode = 0; mode < 2; ++mode) or_gemv(quant, W, quant ? s.data() : nullptr, x.data(), y.data(), rows, cols,
                                                  group, mode);
    }
  auto nw = halves(cols, 1.f);
  std::vector<uint16_t> out(cols);
  or_rmsnorm(x.data(), nw.data(), out.data(), cols, 1e-6f, 0);
  or_rmsnorm(x.data(), nw.data(), out.data(), cols, 1e-6f, 1);
  or_rope(out.data(), 3, 128, 32767, 1e6f);
  const int H = 8, KV = 2, hd = 64, T = 77, stride = 80;
  auto qv = halves((size_t)H * hd, 1.f);
  auto K = halves((size_t)KV * stride * hd, 1.f), V = halves((size_t)KV * stride * hd, 1.f);
  std::vector<uint16_t> att((size_t)H * hd);
  for (int mode = 0; mode < 2; ++mode)
    for (int np : {1, 7, 64}) or_attention(qv.data(), K.data(), V.data(), att.data(), H, KV, hd, stride, T, mode, np);
  std::vector<int8_t> Kq((size_t)KV * stride * hd), Vq((size_t)KV * stride * hd);
  std::vector<float> Ks((size_t)KV * stride), Vs((size_t)KV * stride);
  for (int fmt = 1; fmt <= 2; ++fmt) {
    for (int r = 0; r < KV * stride; ++r) {
      if (fmt == 1) {
        or_quant_row_i8(K.data() + (size_t)r * hd, hd, Kq.data() + (size_t)r * hd, &Ks[r]);
        or_quant_row_i8(V.data() + (size_t)r * hd, hd, Vq.data() + (size_t)r * hd, &Vs[r]);
      } else {
        or_quant_row_f8(K.data() + (size_t)r * hd, hd, reinterpret_cast<uint8_t*>(Kq.data()) + (size_t)r * hd, &Ks[r]);
        or_quant_row_f8(V.data() + (size_t)r * hd, hd, reinterpret_cast<uint8_t*>(Vq.data()) + (size_t)r * hd, &Vs[r]);
      }
    }
    for (int mode = 0; mode < 2; ++mode)
      or_attention_kvq(qv.data(), Kq.data(), Ks.data(), Vq.data(), Vs.data(), att.data(), H, KV, hd, stride, T, mode,
                       64, fmt);
  }
  std::vector<uint8_t> codes(256);
  std::vector<float> vals(256);
  for (int i = 0; i < 256; ++i) codes[i] = (uint8_t)i;
  or_e4m3_decode(codes.data(), 256, vals.data());
  std::vector<float> xs = {0.f, -0.f, 448.f, -448.f, 1e9f, -1e9f, 1e-9f, 3.5f, 0.0009765625f};
  std::vector<uint8_t> enc(xs.size());
  or_e4m3_encode(xs.data(), (int64_t)xs.size(), enc.data());
  auto logits = halves(5000, 3.f);
  std::vector<int> hist = {1, 1, 4999, 0, 77, 4999};
  or_penalty(logits.data(), hist.data(), (int)hist.size(), 5000, 1.1f);
  CHECK(or_argmax(logits.data(), 5000) >= 0);
}

static void write_file(const std::string& p, const std::vector<char>& bytes) {
  FILE* f = std::fopen(p.c_str(), "wb");
  if (!f) return;
  std::fwrite(bytes.data(), 1, bytes.size(), f);
  std::fclose(f);
}
static std::vector<char> read_file(const std::string& p) {
  std::vector<char> b;
  FILE* f = std::fopen(p.c_str(), "rb");
  if (!f) return b;
  std::fseek(f, 0, SEEK_END);
  b.resize((size_t)std::ftell(f));
  std::fseek(f, 0, SEEK_SET);
  if (std::fread(b.data(), 1, b.size(), f) != b.size()) b.clear();
  std::fclose(f);
  return b;
}

static void models(const std::string& dir) {
  struct Case { int quant, lm_fmt, tied; };
  const Case cases[] = {{0, 0, 1}, {0, 0, 0}, {1, 1, 0}, {2, 1, 0}, {2, 0, 1}, {1, 0, 1}};
  for (const Case& c : cases) {
    cq_config cfg{};
    cfg.vocab_size = 512; cfg.dim = 256; cfg.intermediate_size = 384; cfg.n_layers = 2; cfg.n_heads = 4;
    cfg.n_kv_heads = 2; cfg.head_dim = 64; cfg.max_seq_len = 64; cfg.quant_type = c.quant;
    cfg.lm_head_fmt = c.lm_fmt; cfg.tied = c.tied; cfg.norm_eps = 1e-6f; cfg.rope_theta = 1e6f;
    cfg.repetition_penalty = 1.1f;
    const std::string path = dir + "/m" + std::to_string(c.quant) + std::to_string(c.lm_fmt) + std::to_string(c.tied);
    CHECK(cq_write_synthetic_file(path.c_str(), &cfg, 99) == CQ_OK);
    cq_config hdr{};
    CHECK(cq_read_header(path.c_str(), &hdr) == CQ_OK);
    CHECK(hdr.dim == 256 && hdr.tied == c.tied);
    const int cfg11[11] = {cfg.vocab_size, cfg.dim, cfg.intermediate_size, cfg.n_layers, cfg.n_heads,
                           cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len, c.quant, c.lm_fmt, c.tied};
    void* ms = or_model_synth(cfg11, 99, 32);
    void* ml = or_model_load(path.c_str(), 32);
    CHECK(ms && ml);
    if (!ms || !ml) continue;
    std::vector<int> hist;
    int tok = 3;
    for (int pos = 0; pos < 6; ++pos) {
      const int a = or_model_forward(ms, tok, pos, hist.data(), (int)hist.size(), pos & 1);
      const int b = or_model_forward(ml, tok, pos, hist.data(), (int)hist.size(), pos & 1);
      CHECK(a == b);
      hist.push_back(a);
      tok = a;
    }
    CHECK(or_model_forward(ms, 512, 0, nullptr, 0, 0) < 0);   // token out of range
    CHECK(or_model_forward(ms, 1, 32, nullptr, 0, 0) < 0);    // position out of range
    std::vector<uint16_t> lg(512);
    or_model_logits(ms, lg.data());
    const int64_t n = or_model_tensor(ms, 0, 4, 0, nullptr);
    std::vector<uint8_t> t((size_t)n);
    or_model_tensor(ms, 0, 4, 0, t.data());
    for (int kv8 = 1; kv8 <= 2; ++kv8) {
      or_model_set_kv8(ms, kv8);
      or_model_fill_kv(ms, 10, 5);
      or_model_set_nparts(ms, 3);
      or_model_forward(ms, 7, 10, nullptr, 0, 0);
    }
    or_model_free(ms);
    or_model_free(ml);
    // truncated and corrupted copies are rejected by both readers
    const std::vector<char> bytes = read_file(path);
    for (size_t cut : {(size_t)0, (size_t)10, (size_t)256, bytes.size() / 2, bytes.size() - 1}) {
      write_file(path + ".cut", std::vector<char>(bytes.begin(), bytes.begin() + (long)cut));
      void* m = or_model_load((path + ".cut").c_str(), 8);
      if (cut < bytes.size() / 2 || c.lm_fmt == 1) CHECK(m == nullptr);
      if (m) or_model_free(m);
      cq_config h2{};
      const int rc = cq_read_header((path + ".cut").c_str(), &h2);
      if (cut < 256) CHECK(rc != CQ_OK);
    }
    std::vector<char> bad = bytes;
    bad[0] ^= 0x5a;
    write_file(path + ".bad", bad);
    cq_config h3{};
    CHECK(cq_read_header((path + ".bad").c_str(), &h3) == CQ_EFORMAT);
    CHECK(or_model_load((path + ".bad").c_str(), 8) == nullptr);
  }
  cq_config bad{};
  CHECK(cq_write_synthetic_file((dir + "/x").c_str(), &bad, 1) != CQ_OK);
  CHECK(cq_read_header((dir + "/does_not_exist").c_str(), &bad) == CQ_EIO);
  for (const char* m : {"0.5B", "1.5B", "3B", "7B", "14B"})
    for (int q = 0; q <= 2; ++q) {
      cq_config p{};
      CHECK(cq_config_preset(m, q, &p) == CQ_OK);
    }
  cq_config p{};
  CHECK(cq_config_preset("13B", 0, &p) != CQ_OK);
  CHECK(cq_config_preset("7B", 3, &p) != CQ_OK);
}

static void tokenizer(const std::string& dir) {
  // a small ranks file: byte alphabet entries, merges, escapes, a surrogate pair, added tokens
  std::string json = "{\"vocab\": {";
  const char* toks[] = {"a", "b", "c", "ab", "abc", "\\u0120", "\\u0120a", "\\u00e9", "\\ud83d\\ude00", "\\\"q\\\"",
                        "<|endoftext|>"};
  for (int i = 0; i < 11; ++i) json += std::string(i ? ", " : "") + "\"" + toks[i] + "\": " + std::to_string(i);
  json += "}, \"special_tokens\": {\"eos_token\": \"<|endoftext|>\", \"list\": [1, {\"x\": null}, true]}, "
          "\"added_tokens\": {\"10\": \"<|endoftext|>\", \"11\": \"<|im_start|>\", \"12\": \"<|im_end|>\"}}";
  const std::string path = dir + "/ranks.json";
  write_file(path, std::vector<char>(json.begin(), json.end()));
  cq_tokenizer* t = nullptr;
  CHECK(cq_tokenizer_load(path.c_str(), &t) == CQ_OK);
  if (!t) return;
  std::uniform_int_distribution<int> byte(0, 255), len(0, 200);
  std::vector<int32_t> ids(4096);
  std::vector<char> buf(1 << 16);
  for (int it = 0; it < 2000; ++it) {
    std::string s;
    const int n = len(rng);
    for (int i = 0; i < n; ++i) {
      const int r = byte(rng);
      if (r < 8) s += "<|im_end|>";
      else if (r < 12) s += "\xf0\x9f\x98\x80";
      else if (r < 40) s += "ab c";
      else s += (char)byte(rng);
    }
    int32_t nout = 0;
    int rc = cq_tokenizer_encode(t, s.data(), s.size(), ids.data(), 3, &nout);   // too small first
    if (rc == CQ_ERANGE) rc = cq_tokenizer_encode(t, s.data(), s.size(), ids.data(), (int32_t)ids.size(), &nout);
    CHECK(rc == CQ_OK);
    size_t blen = 0;
    rc = cq_tokenizer_decode(t, ids.data(), nout, buf.data(), 2, &blen);
    if (rc == CQ_ERANGE) rc = cq_tokenizer_decode(t, ids.data(), nout, buf.data(), buf.size(), &blen);
    CHECK(rc == CQ_OK);
  }
  int32_t bogus[3] = {-5, 1 << 30, 4};
  size_t blen = 0;
  CHECK(cq_tokenizer_decode(t, bogus, 3, buf.data(), buf.size(), &blen) == CQ_OK);
  CHECK(cq_tokenizer_token_id(t, "<|im_end|>") == 12);
  CHECK(cq_tokenizer_vocab_size(t) == 13);
  cq_tokenizer_free(t);
  const char* roles[] = {"system", "user", "assistant"};
  const char* contents[] = {"be brief", "hi \xff there", ""};
  size_t need = 0;
  CHECK(cq_chat_template(roles, contents, 3, 1, buf.data(), 4, &need) == CQ_ERANGE);
  CHECK(cq_chat_template(roles, contents, 3, 1, buf.data(), buf.size(), &need) == CQ_OK);
  // malformed ranks files are rejected
  const char* bad[] = {"", "{", "{\"vocab\": {\"a\": }}", "{\"vocab\": {\"a\": 1", "{\"vocab\": {\"\\ud800\": 1}}",
                       "{\"added_tokens\": {\"x\": \"y\"}}", "[1, 2]", "{\"vocab\": {\"a\": -1}}",
                       "{\"vocab\": {\"a\": 99999999999}}", "{\"vocab\": {\"a\": \"1\"}}", "{\"vocab\": {}}"};
  for (const char* b : bad) {
    write_file(path, std::vector<char>(b, b + std::strlen(b)));
    cq_tokenizer* u = nullptr;
    CHECK(cq_tokenizer_load(path.c_str(), &u) != CQ_OK);
    cq_tokenizer_free(u);
  }
}

int main(int argc, char** argv) {
  const std::string dir = argc > 1 ? argv[1] : ".";
  oracle_ops();
  models(dir);
  tokenizer(dir);
  if (g_fail) {
    std::fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  std::printf("sanitize ok\n");
  return 0;
}
