// Host side of the weight format: presets, header validation, the
// exporter's quantizer and the synthetic weight-file writer.
#include "cq_format.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>

namespace cq {

static thread_local std::string g_error;
void set_error(const std::string& msg) { g_error = msg; }
int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

// ------------------------------------------------------------------ presets
// include/config.h:55-113 (model values), :124-126 (eps, theta, penalty).
struct Preset {
  const char* name;
  int vocab, dim, inter, layers, heads, kv, hd;
  bool tied;   // tie_word_embeddings of the checkpoint the preset describes
};
static const Preset kPresets[] = {
    {"0.5B", 151936, 896, 4864, 24, 14, 2, 64, true},
    {"1.5B", 151936, 1536, 8960, 28, 12, 2, 128, true},
    {"3B", 151936, 2048, 11008, 36, 16, 2, 128, true},
    {"7B", 152064, 3584, 18944, 28, 28, 4, 128, false},
    {"14B", 152064, 5120, 13824, 48, 40, 8, 128, false},
};

int validate_config(const cq_config& c) {
  if (c.vocab_size <= 0 || c.dim <= 0 || c.intermediate_size <= 0 || c.n_layers <= 0 || c.n_heads <= 0 ||
      c.n_kv_heads <= 0 || c.head_dim <= 0 || c.max_seq_len <= 0)
    return fail(CQ_EFORMAT, "config: non-positive dimension");
  if (c.quant_type < 0 || c.quant_type > 2) return fail(CQ_EFORMAT, "config: unknown quant type");
  if (c.lm_head_fmt != CQ_LMHEAD_FP16 && c.lm_head_fmt != CQ_LMHEAD_INT8)
    return fail(CQ_EFORMAT, "config: unknown lm_head format");
  if (c.lm_head_fmt == CQ_LMHEAD_INT8 && c.tied) return fail(CQ_EFORMAT, "config: an int8 lm_head cannot be tied");
  if (c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 16)
    return fail(CQ_EINVAL, "config: n_heads must be a multiple of n_kv_heads with a group of at most 16");
  if (c.head_dim != 64 && c.head_dim != 128) return fail(CQ_EINVAL, "config: head_dim must be 64 or 128");
  if (c.dim % kGroup || c.intermediate_size % kGroup || (c.n_heads * c.head_dim) % kGroup)
    return fail(CQ_EINVAL, "config: dim, intermediate_size and n_heads*head_dim must be multiples of 128");
  if (c.max_seq_len % 32) return fail(CQ_EINVAL, "config: max_seq_len must be a multiple of 32");
  if (c.n_kv_heads > 64) return fail(CQ_EINVAL, "config: at most 64 kv heads");
  return CQ_OK;
}

static int64_t qbytes(int quant, int64_t rows, int64_t cols) { return rows * row_bytes(quant, cols); }

std::vector<TensorSpec> tensor_list(const cq_config& c) {
  std::vector<TensorSpec> v;
  const int64_t d = c.dim, I = c.intermediate_size, qd = (int64_t)c.n_heads * c.head_dim,
                kvd = (int64_t)c.n_kv_heads * c.head_dim;
  const int qt = c.quant_type;
  auto vec = [&](int kind, int layer, int64_t n) {
    v.push_back({kind, layer, 1, n, CQ_QUANT_FP16, n * 2, 0});
  };
  auto proj = [&](int kind, int layer, int64_t rows, int64_t cols, int quant) {
    v.push_back({kind, layer, rows, cols, quant, qbytes(quant, rows, cols),
                 quant == CQ_QUANT_FP16 ? 0 : rows * (cols / kGroup) * 2});
  };
  proj(TK_EMBED, -1, c.vocab_size, d, CQ_QUANT_FP16);
  for (int l = 0; l < c.n_layers; ++l) {
    vec(TK_IN_NORM, l, d);
    proj(TK_WQ, l, qd, d, qt);
    vec(TK_BQ, l, qd);
    proj(TK_WK, l, kvd, d, qt);
    vec(TK_BK, l, kvd);
    proj(TK_WV, l, kvd, d, qt);
    vec(TK_BV, l, kvd);
    proj(TK_WO, l, d, qd, qt);
    vec(TK_POST_NORM, l, d);
    proj(TK_WG, l, I, d, qt);
    proj(TK_WU, l, I, d, qt);
    proj(TK_WD, l, d, I, qt);
  }
  vec(TK_FINAL_NORM, -1, d);
  if (c.lm_head_fmt == CQ_LMHEAD_INT8) proj(TK_LM_HEAD, -1, c.vocab_size, d, CQ_QUANT_INT8);
  else if (!c.tied) proj(TK_LM_HEAD, -1, c.vocab_size, d, CQ_QUANT_FP16);
  return v;
}

int64_t file_bytes(const cq_config& c) {
  int64_t n = 256;
  for (const auto& t : tensor_list(c)) n += t.weight_bytes + t.scale_bytes;
  return n;
}

float kind_mean(int kind) {
  return (kind == TK_IN_NORM || kind == TK_POST_NORM || kind == TK_FINAL_NORM) ? 1.0f : 0.0f;
}

// --------------------------------------------------------------- quantizer
// export_weights.py:123-146 (int8) and :161-183 (int4): per group of `group`
// consecutive weights of a row, s = max|w| / qmax in fp32 (w widened from
// fp16), q = clip(round_half_even(w / (s > 0 ? s : 1)), -qmax, qmax), the
// stored scale is fp16(s).  Int4 packs element 2p in the low nibble and 2p+1
// in the high nibble of byte p (export_weights.py:197-199).
void quantize_host(int quant, const uint16_t* w, int64_t rows, int64_t cols, int group, uint8_t* q, uint16_t* s) {
  const float qmax = quant == CQ_QUANT_INT4 ? 7.0f : 127.0f;
  const int64_t g = group > 0 ? group : cols;
  const int64_t ng = cols / g;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t gi = 0; gi < ng; ++gi) {
      const uint16_t* wg = w + r * cols + gi * g;
      float mx = 0.f;
      for (int64_t i = 0; i < g; ++i) mx = std::fmax(mx, std::fabs(h2f_bits(wg[i])));
      const float sc = mx / qmax;
      const float safe = sc > 0.f ? sc : 1.0f;
      s[r * ng + gi] = f2h_bits(sc);
      for (int64_t i = 0; i < g; ++i) {
        float v = std::nearbyint(h2f_bits(wg[i]) / safe);
        v = std::fmin(std::fmax(v, -qmax), qmax);
        const int qi = (int)v;
        const int64_t col = gi * g + i;
        if (quant == CQ_QUANT_INT8) {
          q[r * cols + col] = (uint8_t)(int8_t)qi;
        } else {
          uint8_t& b = q[r * (cols / 2) + col / 2];
          const uint8_t nib = (uint8_t)(qi & 0xF);
          if (col & 1) b = (uint8_t)((b & 0x0F) | (nib << 4));
          else b = (uint8_t)((b & 0xF0) | nib);
        }
      }
    }
  }
}

void synth_tensor_host(uint64_t seed, const TensorSpec& t, std::vector<uint16_t>& out) {
  const int64_t n = t.rows * t.cols;
  out.resize((size_t)n);
  const uint64_t stream = tensor_stream(t.layer, t.kind);
  const float mul = synth_mul(kWeightSigma), mean = kind_mean(t.kind);
  for (int64_t i = 0; i < n; ++i) out[(size_t)i] = synth_half(seed, stream, (uint64_t)i, mul, mean);
}

}  // namespace cq

// ===================================================================== C ABI
using namespace cq;

extern "C" const char* cq_last_error(void) { return g_error.c_str(); }

extern "C" int cq_config_preset(const char* model, int32_t quant_type, cq_config* out) {
  if (!model || !out) return fail(CQ_EINVAL, "preset: null argument");
  if (quant_type < 0 || quant_type > 2) return fail(CQ_EINVAL, "preset: unknown quant type");
  for (const auto& p : kPresets) {
    if (std::strcmp(p.name, model) == 0) {
      cq_config c{};
      c.vocab_size = p.vocab;
      c.dim = p.dim;
      c.intermediate_size = p.inter;
      c.n_layers = p.layers;
      c.n_heads = p.heads;
      c.n_kv_heads = p.kv;
      c.head_dim = p.hd;
      c.max_seq_len = 32768;
      c.quant_type = quant_type;
      // export_weights.py:261: a separate lm_head is int8 in quantized builds
      c.tied = p.tied ? 1 : 0;
      c.lm_head_fmt = (!p.tied && quant_type != CQ_QUANT_FP16) ? CQ_LMHEAD_INT8 : CQ_LMHEAD_FP16;
      c.norm_eps = 1e-6f;
      c.rope_theta = 1000000.0f;
      c.repetition_penalty = 1.1f;
      *out = c;
      return CQ_OK;
    }
  }
  return fail(CQ_EINVAL, std::string("preset: unknown model '") + model + "'");
}

extern "C" int cq_read_header(const char* path, cq_config* cfg) {
  if (!path || !cfg) return fail(CQ_EINVAL, "read_header: null argument");
  FILE* f = std::fopen(path, "rb");
  if (!f) return fail(CQ_EIO, std::string("cannot open weight file: ") + path);
  int32_t h[11] = {0};
  const size_t got = std::fread(h, sizeof(int32_t), 11, f);
  std::fseek(f, 0, SEEK_END);
  const long end = std::ftell(f);
  std::fclose(f);
  if (got != 11) return fail(CQ_EIO, "failed to read the weight header");
  if (h[0] != CQ_MAGIC) {
    char b[96];
    std::snprintf(b, sizeof b, "magic number mismatch: expected 0x%X, found 0x%X", CQ_MAGIC, (unsigned)h[0]);
    return fail(CQ_EFORMAT, b);
  }
  cq_config c{};
  c.vocab_size = h[1];
  c.dim = h[2];
  c.intermediate_size = h[3];
  c.n_layers = h[4];
  c.n_heads = h[5];
  c.n_kv_heads = h[6];
  c.head_dim = h[7];
  c.max_seq_len = h[8];
  c.quant_type = h[9];
  c.lm_head_fmt = h[10];
  c.norm_eps = 1e-6f;
  c.rope_theta = 1000000.0f;
  c.repetition_penalty = 1.1f;
  c.tied = 0;
  CQ_TRY(validate_config(c));
  // load_weights.cpp:139-161: without an int8 lm_head, an fp16 lm_head is
  // present iff the bytes left after final_norm hold V*d halves.
  if (c.lm_head_fmt == CQ_LMHEAD_FP16) {
    c.tied = 1;
    const int64_t tied_bytes = file_bytes(c);
    if ((int64_t)end - tied_bytes >= (int64_t)c.vocab_size * c.dim * 2) c.tied = 0;
  }
  if ((int64_t)end < file_bytes(c)) return fail(CQ_EIO, "weight file is truncated");
  *cfg = c;
  return CQ_OK;
}

extern "C" int cq_quantize(int32_t quant_type, const uint16_t* w, int64_t rows, int64_t cols, int32_t group,
                           void* q_out, uint16_t* s_out) {
  if (quant_type != CQ_QUANT_INT8 && quant_type != CQ_QUANT_INT4) return fail(CQ_EINVAL, "quantize: int8/int4 only");
  if (!w || !q_out || !s_out || rows <= 0 || cols <= 0) return fail(CQ_EINVAL, "quantize: bad arguments");
  if (group < 0 || (group > 0 && cols % group) || (quant_type == CQ_QUANT_INT4 && cols % 2))
    return fail(CQ_EINVAL, "quantize: cols must be a multiple of the group (and even for int4)");
  quantize_host(quant_type, w, rows, cols, group, (uint8_t*)q_out, s_out);
  return CQ_OK;
}

extern "C" int cq_write_synthetic_file(const char* path, const cq_config* cfg, uint64_t seed) {
  if (!path || !cfg) return fail(CQ_EINVAL, "write: null argument");
  CQ_TRY(validate_config(*cfg));
  FILE* f = std::fopen(path, "wb");
  if (!f) return fail(CQ_EIO, std::string("cannot create ") + path);
  // export_weights.py:270-279: 11 int32 then zero padding to 256 bytes.
  int32_t h[64] = {0};
  h[0] = CQ_MAGIC;
  h[1] = cfg->vocab_size;
  h[2] = cfg->dim;
  h[3] = cfg->intermediate_size;
  h[4] = cfg->n_layers;
  h[5] = cfg->n_heads;
  h[6] = cfg->n_kv_heads;
  h[7] = cfg->head_dim;
  h[8] = cfg->max_seq_len;
  h[9] = cfg->quant_type;
  h[10] = cfg->lm_head_fmt;
  bool ok = std::fwrite(h, 1, 256, f) == 256;
  std::vector<uint16_t> vals;
  std::vector<uint8_t> q;
  std::vector<uint16_t> s;
  for (const auto& t : tensor_list(*cfg)) {
    if (!ok) break;
    synth_tensor_host(seed, t, vals);
    if (t.quant == CQ_QUANT_FP16) {
      ok = std::fwrite(vals.data(), 2, vals.size(), f) == vals.size();
    } else {
      q.assign((size_t)t.weight_bytes, 0);
      s.assign((size_t)(t.scale_bytes / 2), 0);
      quantize_host(t.quant, vals.data(), t.rows, t.cols, kGroup, q.data(), s.data());
      ok = std::fwrite(q.data(), 1, q.size(), f) == q.size() && std::fwrite(s.data(), 2, s.size(), f) == s.size();
    }
  }
  if (std::fclose(f) != 0) ok = false;
  if (!ok) return fail(CQ_EIO, std::string("short write to ") + path);
  return CQ_OK;
}

extern "C" uint16_t cq_synth_normal(uint64_t seed, uint64_t stream, uint64_t index, float sigma) {
  return synth_half(seed, stream, index, synth_mul(sigma), 0.f);
}
extern "C" uint32_t cq_synth_uniform(uint64_t seed, uint64_t stream, uint64_t index, uint32_t n) {
  return n ? (uint32_t)(rand64(seed, stream, index) % n) : 0u;
}
extern "C" uint64_t cq_tensor_stream_id(int32_t layer, int32_t kind) { return tensor_stream(layer, kind); }
extern "C" uint64_t cq_kv_stream_id(int32_t layer, int32_t kv_head, int32_t kind) {
  return kv_stream(layer, kv_head, kind);
}
extern "C" int64_t cq_kv_k_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim) {
  return kv_k_offset(kv_head, t, d, max_seq_len, head_dim);
}
extern "C" int64_t cq_kv_v_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim) {
  return kv_v_offset(kv_head, t, d, max_seq_len, head_dim);
}
extern "C" int64_t cq_kv8_k_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim) {
  return cq::kv8_k_offset(kv_head, t, d, max_seq_len, head_dim);
}
extern "C" int64_t cq_kv8_v_offset(int32_t kv_head, int32_t t, int32_t d, int32_t max_seq_len, int32_t head_dim) {
  return cq::kv8_v_offset(kv_head, t, d, max_seq_len, head_dim);
}
