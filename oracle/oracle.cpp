// Scalar host C++ oracle of the CuQwen batch-1 decode path.
//
// TEST INFRASTRUCTURE ONLY: this file is the checker for the HIP library.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
// it; the product never does.  It shares no code with the product: it has
// its own fp16 conversion, its own format reader and its own restatement of
// the synthetic generator.
//
// Each function cites the reference file:line it restates
// (talhatahir-10xe/CuQwen, paths relative to its root).  Two modes:
//   mode 0 ("ref-rounding"): fp16 rounding at exactly the reference's
//           points (q/k/v, RoPE output, residual, RMSNorm output, SwiGLU
//           output, scores and P in attention, attention output, logits),
//           fp32 accumulation in the reference's lane order;
//   mode 1 ("fp32"): the same graph with double accumulation and no
//           rounding of scores / P, the yardstick for the 1e-2 tolerance.
//
// Build: oracle/Makefile (g++ -O2 -fopenmp -shared).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include <omp.h>

#include <chrono>

namespace {

// ------------------------------------------------------------------ fp16
float h2f_bits(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  const uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) bits = sign;
    else {  // subnormal: man * 2^-24
      float f = (float)man * 5.9604644775390625e-08f;
      uint32_t b;
      std::memcpy(&b, &f, 4);
      bits = sign | b;
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// All 65536 conversions, tabulated once (exact: the table holds h2f_bits).
struct H2FTable {
  float v[65536];
  H2FTable() {
    for (uint32_t i = 0; i < 65536; ++i) v[i] = h2f_bits((uint16_t)i);
  }
};
const H2FTable kH2F;   // built when the library loads
inline float h2f(uint16_t h) { return kH2F.v[h]; }

// float -> fp16, round to nearest even (IEEE 754 binary16).
uint16_t f2h(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00 : 0x7C00);   // nan / inf
  if (ax >= 0x477FF000u) return sign | 0x7C00;   // rounds to >= 65520 -> inf
  if (ax < 0x38800000u) {   // below 2^-14: subnormal or zero
    // value in units of 2^-24, rounded half to even
    float a;
    std::memcpy(&a, &ax, 4);
    const double u = (double)a * 16777216.0;
    double r = std::nearbyint(u);   // default rounding mode: half to even
    return sign | (uint16_t)r;
  }
  const uint32_t e = (ax >> 23) - 112;
  uint32_t m = ax & 0x7FFFFF;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h += 1;   // carries into the exponent correctly
  return sign | (uint16_t)h;
}
inline float rh(float f) { return h2f(f2h(f)); }   // round through fp16

// ------------------------------------------------------------- generator
// Restatement of the synthetic input generator (splitmix64 finaliser,
// Irwin-Hall sum of four 16-bit uniforms, sd 37836.51).
uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
uint64_t rnd(uint64_t seed, uint64_t stream, uint64_t index) {
  const uint64_t key = mix64(seed + 0x9E3779B97F4A7C15ull * (stream + 1));
  return mix64(key + 0x9E3779B97F4A7C15ull * (index + 1));
}
uint16_t gen_half(uint64_t seed, uint64_t stream, uint64_t index, float mul, float mean) {
  const uint64_t r = rnd(seed, stream, index);
  const int32_t s = (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) + (int32_t)((r >> 32) & 0xFFFF) +
                    (int32_t)((r >> 48) & 0xFFFF) - 131070;
  volatile float v = (float)s * mul;   // separately rounded multiply, then add
  return f2h(v + mean);
}
float gen_mul(double sigma) { return (float)(sigma / 37836.51); }
uint64_t tensor_stream(int layer, int kind) { return (uint64_t)(layer + 1) * 32u + (uint64_t)kind; }
uint64_t kv_stream(int layer, int kv_head, int kind) {
  return 0x100000000ull + ((uint64_t)layer * 4096u + (uint64_t)kv_head) * 2u + (uint64_t)kind;
}
enum { K_EMBED = 0, K_FINAL_NORM = 1, K_LM_HEAD = 2, K_IN_NORM = 3, K_WQ = 4, K_BQ = 5, K_WK = 6, K_BK = 7,
       K_WV = 8, K_BV = 9, K_WO = 10, K_POST_NORM = 11, K_WG = 12, K_WU = 13, K_WD = 14 };

// ------------------------------------------------------------- quantizer
// export_weights.py:123-146 (int8), :161-205 (int4 + packing).
void quantize(int quant, const uint16_t* w, int64_t rows, int64_t cols, int64_t group, uint8_t* q, uint16_t* s) {
  const float qmax = quant == 2 ? 7.0f : 127.0f;
  const int64_t g = group > 0 ? group : cols, ng = cols / g;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t gi = 0; gi < ng; ++gi) {
      float mx = 0.f;
      for (int64_t i = 0; i < g; ++i) {
        const float a = std::fabs(h2f(w[r * cols + gi * g + i]));
        if (a > mx) mx = a;
      }
      const float sc = mx / qmax;                   // np.max(abs) / 127.0 in fp32
      const float safe = sc > 0.f ? sc : 1.0f;      // np.where(scales > 0, scales, 1)
      s[r * ng + gi] = f2h(sc);                     // scales.astype(np.float16)
      for (int64_t i = 0; i < g; ++i) {
        const int64_t col = gi * g + i;
        float v = std::nearbyint(h2f(w[r * cols + col]) / safe);   // np.round: half to even
        if (v > qmax) v = qmax;
        if (v < -qmax) v = -qmax;
        const int qi = (int)v;
        if (quant == 1) q[r * cols + col] = (uint8_t)(int8_t)qi;
        else {
          uint8_t& b = q[r * (cols / 2) + col / 2];
          const uint8_t nib = (uint8_t)(qi & 0xF);   // (q & 0xF), export_weights.py:198
          b = (col & 1) ? (uint8_t)((b & 0x0F) | (nib << 4)) : (uint8_t)((b & 0xF0) | nib);
        }
      }
    }
}

// ------------------------------------------------------------------ dot8
// kernels.cu:11-57: one 8-element chunk c of a row, nested fma order
// p = fma(b[2k], x[2k], fma(b[2k+1], x[2k+1], p)) for k = 0..3, times the
// chunk's scale (index c >> 4 for group 128).
float dot8(int quant, const uint8_t* wrow, const uint16_t* srow, int64_t c, const uint16_t* x, int64_t group) {
  float b[8];
  if (quant == 0) {
    const uint16_t* w = reinterpret_cast<const uint16_t*>(wrow) + 8 * c;
    for (int i = 0; i < 8; ++i) b[i] = h2f(w[i]);
  } else if (quant == 1) {
    for (int i = 0; i < 8; ++i) b[i] = (float)(int8_t)wrow[8 * c + i];
  } else {
    for (int k = 0; k < 4; ++k) {
      const int byte = wrow[4 * c + k];
      b[2 * k] = (float)(((byte & 0xF) ^ 0x8) - 0x8);            // low nibble -> element 2k
      b[2 * k + 1] = (float)((((byte >> 4) & 0xF) ^ 0x8) - 0x8); // high nibble -> 2k+1
    }
  }
  float p = 0.f;
  for (int k = 0; k < 4; ++k)
    p = std::fma(b[2 * k], h2f(x[8 * c + 2 * k]), std::fma(b[2 * k + 1], h2f(x[8 * c + 2 * k + 1]), p));
  if (quant == 0) return p;
  const int64_t gi = group > 0 ? (8 * c) / group : 0;
  return p * h2f(srow[gi]);
}

int64_t row_bytes(int quant, int64_t cols) { return quant == 2 ? cols / 2 : quant == 1 ? cols : 2 * cols; }

// One GEMV row.  mode 0: 32 lanes accumulate chunks c = lane, lane+32, ...
// then a shfl_down tree (kernels.cu:458-466).  mode 1: double sum.
float gemv_row(int quant, const uint8_t* W, const uint16_t* S, const uint16_t* x, int64_t row, int64_t cols,
               int64_t group, int mode) {
  const uint8_t* wrow = W + row * row_bytes(quant, cols);
  const int64_t ng = group > 0 ? cols / group : 1;
  const uint16_t* srow = S ? S + row * ng : nullptr;
  const int64_t nc = cols / 8;
  if (mode == 1) {
    double acc = 0.0;
    for (int64_t c = 0; c < nc; ++c) {
      double p = 0.0;
      for (int i = 0; i < 8; ++i) {
        double w;
        const int64_t e = 8 * c + i;
        if (quant == 0) w = h2f(reinterpret_cast<const uint16_t*>(wrow)[e]);
        else if (quant == 1) w = (int8_t)wrow[e];
        else {
          const int byte = wrow[e / 2];
          const int n = (e & 1) ? (byte >> 4) & 0xF : byte & 0xF;
          w = (double)((n ^ 8) - 8);
        }
        p += w * h2f(x[e]);
      }
      if (quant != 0) p *= h2f(srow[group > 0 ? (8 * c) / group : 0]);
      acc += p;
    }
    return (float)acc;
  }
  // lane l adds chunks l, l+32, l+64, ... in that order; the 32 lanes'
  // chains are interleaved (independent, so the host overlaps them)
  float lanes[32] = {0.f};
  for (int64_t c0 = 0; c0 < nc; c0 += 32) {
    const int n = (int)std::min<int64_t>(32, nc - c0);
    for (int l = 0; l < n; ++l) lanes[l] += dot8(quant, wrow, srow, c0 + l, x, group);
  }
  for (int off = 16; off > 0; off >>= 1)
    for (int l = 0; l < off; ++l) lanes[l] += lanes[l + off];
  return lanes[0];
}

// --------------------------------------------------------------- rmsnorm
// kernels.cu:689-751: out = half((x * rsqrt(mean(x^2) + half(eps))) * w).
void rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int64_t dim, float eps, int mode) {
  double ss = 0.0;
  for (int64_t i = 0; i < dim; ++i) ss += (double)h2f(x[i]) * h2f(x[i]);
  const float epsh = h2f(f2h(eps));
  const float inv = mode == 1 ? (float)(1.0 / std::sqrt(ss / dim + epsh)) : 1.0f / std::sqrt((float)ss / (float)dim + epsh);
  for (int64_t i = 0; i < dim; ++i) out[i] = f2h((h2f(x[i]) * inv) * h2f(w[i]));
}

// ------------------------------------------------------------------ rope
// kernels.cu:370-398: NeoX rotation of (i, i + hd/2), freq = theta^(-2i/hd),
// angle = pos * freq -- evaluated in double (the reference's fast-math
// sinf/cosf are approximate at large angles).
void rope(uint16_t* v, int n_heads, int hd, int pos, float theta) {
  const int half = hd / 2;
  for (int h = 0; h < n_heads; ++h)
    for (int i = 0; i < half; ++i) {
      const double freq = 1.0 / std::pow((double)theta, (2.0 * i) / (double)hd);
      const double ang = (double)pos * freq;
      const float c = (float)std::cos(ang), s = (float)std::sin(ang);
      const float v0 = h2f(v[h * hd + i]), v1 = h2f(v[h * hd + i + half]);
      const float a = v0 * c, b = v1 * s, cc = v1 * c, d = v0 * s;
      v[h * hd + i] = f2h(a - b);
      v[h * hd + i + half] = f2h(cc + d);
    }
}

// ------------------------------------------------------------- attention
// K/V head-major [n_kv][stride][hd] fp16 (model.cu:112-114), keys [0, T).
// mode 0: the reference's split-K semantics (kernels.cu:105-288) with
// `nparts` partitions of ceil(T/nparts) keys: scores rounded to fp16 after
// the 1/sqrt(hd) scale, e = exp(s - m_part) rounded to fp16 for P*V while the
// partition sum adds the unrounded e, then the log-sum-exp merge with
// 1/(L + 1e-9).  mode 1: softmax(q.k/sqrt(hd)) v in double.
void attention(const uint16_t* q, const uint16_t* K, const uint16_t* V, uint16_t* out, int n_heads, int n_kv,
               int hd, int64_t stride, int T, int mode, int nparts) {
  const int g = n_heads / n_kv;
  const float scale = 1.0f / std::sqrt((float)hd);
#pragma omp parallel for schedule(dynamic)
  for (int h = 0; h < n_heads; ++h) {
    const int kvh = h / g;
    const uint16_t* qh = q + (int64_t)h * hd;
    const uint16_t* Kh = K + (int64_t)kvh * stride * hd;
    const uint16_t* Vh = V + (int64_t)kvh * stride * hd;
    std::vector<double> s(T);
    if (mode == 1) {
      double mx = -INFINITY;
      for (int t = 0; t < T; ++t) {
        double a = 0.0;
        for (int d = 0; d < hd; ++d) a += (double)h2f(qh[d]) * h2f(Kh[(int64_t)t * hd + d]);
        s[t] = a / std::sqrt((double)hd);
        if (s[t] > mx) mx = s[t];
      }
      double L = 0.0;
      std::vector<double> o(hd, 0.0);
      for (int t = 0; t < T; ++t) {
        const double e = std::exp(s[t] - mx);
        L += e;
        for (int d = 0; d < hd; ++d) o[d] += e * h2f(Vh[(int64_t)t * hd + d]);
      }
      for (int d = 0; d < hd; ++d) out[(int64_t)h * hd + d] = f2h((float)(o[d] / L));
      continue;
    }
    const int chunk = (T + nparts - 1) / nparts;
    const int nonempty = (T + chunk - 1) / chunk;
    std::vector<float> pm(nonempty), ps(nonempty), po((size_t)nonempty * hd);
    for (int p = 0; p < nonempty; ++p) {
      const int t0 = p * chunk, t1 = std::min(t0 + chunk, T);
      std::vector<float> sc(t1 - t0);
      float mx = -1e30f;
      for (int t = t0; t < t1; ++t) {
        float a = 0.f;
        for (int d = 0; d < hd; ++d) a += h2f(qh[d]) * h2f(Kh[(int64_t)t * hd + d]);
        sc[t - t0] = rh(a * scale);
        mx = std::max(mx, sc[t - t0]);
      }
      float sum = 0.f;
      std::vector<float> pv(hd, 0.f);
      for (int t = t0; t < t1; ++t) {
        const float e = std::exp(sc[t - t0] - mx);
        sum += e;
        const float P = rh(e);
        for (int d = 0; d < hd; ++d) pv[d] += P * h2f(Vh[(int64_t)t * hd + d]);
      }
      pm[p] = mx;
      ps[p] = sum;
      for (int d = 0; d < hd; ++d) po[(size_t)p * hd + d] = pv[d];
    }
    float M = -1e30f;
    for (int p = 0; p < nonempty; ++p) M = std::max(M, pm[p]);
    std::vector<float> r(nonempty);
    float L = 0.f;
    for (int p = 0; p < nonempty; ++p) {
      r[p] = std::exp(pm[p] - M);
      L += ps[p] * r[p];
    }
    const float inv = 1.0f / (L + 1e-9f);
    for (int d = 0; d < hd; ++d) {
      float a = 0.f;
      for (int p = 0; p < nonempty; ++p) a += po[(size_t)p * hd + d] * r[p];
      out[(int64_t)h * hd + d] = f2h(a * inv);
    }
  }
}

// ------------------------------------------------------------ int8 KV
// An extension of the reference (its KV cache is fp16, src/model.cu:37-38;
// a quantized cache is its roadmap item, README.md:147): each (position,
// kv head) row of K and of V is stored as q = clamp(rint(x / s), -127, 127)
// with s = max|x| / 127 in fp32 (a zero row keeps s = 0 and q = 0).
void quant_row_i8(const uint16_t* x, int n, int8_t* q, float* s) {
  float amax = 0.f;
  for (int i = 0; i < n; ++i) amax = std::max(amax, std::fabs(h2f(x[i])));
  const float sc = amax / 127.0f;
  *s = sc;
  for (int i = 0; i < n; ++i) {
    if (sc == 0.f) { q[i] = 0; continue; }
    const float r = std::nearbyint(h2f(x[i]) / sc);   // round half to even
    q[i] = (int8_t)std::max(-127.f, std::min(127.f, r));
  }
}

// ------------------------------------------------------------- fp8 KV
// The other format of the same roadmap item (README.md:147, "int8/fp8"):
// OCP FP8 E4M3 ("e4m3fn": sign, 4 exponent bits with bias 7, 3 mantissa
// bits, no infinities, 0x7F / 0xFF are NaN, largest finite 448).  A row is
// stored as q = e4m3(x / s) with s = max|x| / 448 in fp32, rounding to
// nearest with ties to an even mantissa; a zero row keeps s = 0, q = 0.
float e4m3_decode(uint8_t b) {
  const int e = (b >> 3) & 15, m = b & 7;
  float v;
  if (e == 15 && m == 7) v = NAN;
  else if (e == 0) v = std::ldexp((float)m, -9);              // subnormal: m * 2^-9
  else v = std::ldexp(1.0f + (float)m / 8.0f, e - 7);
  return (b & 0x80) ? -v : v;
}

// Finite x to E4M3, round to nearest even, saturating at +-448.
uint8_t e4m3_encode(float x) {
  const uint8_t sign = std::signbit(x) ? 0x80 : 0;
  const float a = std::fabs(x);
  if (a < 0.015625f) {   // below 2^-6: the subnormal grid m * 2^-9 (m = 8 is 2^-6, code 0x08)
    return sign | (uint8_t)std::nearbyint(a * 512.0f);   // exact scaling, round half to even
  }
  int k;
  const float f = std::frexp(a, &k);   // a = f * 2^k, f in [0.5, 1)
  int E = k - 1;                       // a = r * 2^E, r in [1, 2)
  const float r = f * 2.0f;
  int m = (int)std::nearbyint((r - 1.0f) * 8.0f);   // r - 1 and the * 8 are exact
  if (m == 8) { m = 0; ++E; }
  if (E > 8 || (E == 8 && m > 6)) return sign | 0x7E;   // beyond 448
  return sign | (uint8_t)(((E + 7) << 3) | m);
}

void quant_row_f8(const uint16_t* x, int n, uint8_t* q, float* s) {
  float amax = 0.f;
  for (int i = 0; i < n; ++i) amax = std::max(amax, std::fabs(h2f(x[i])));
  const float sc = amax / 448.0f;
  *s = sc;
  for (int i = 0; i < n; ++i) q[i] = sc == 0.f ? 0 : e4m3_encode(h2f(x[i]) / sc);
}

// Value of one stored byte of a quantized cache (before its row scale):
// fmt 1 int8, 2 E4M3.
inline float kv_code(int fmt, int8_t b) { return fmt == 2 ? e4m3_decode((uint8_t)b) : (float)b; }

void quant_row_kv(int fmt, const uint16_t* x, int n, int8_t* q, float* s) {
  if (fmt == 2) quant_row_f8(x, n, reinterpret_cast<uint8_t*>(q), s);
  else quant_row_i8(x, n, q, s);
}

// Attention over a quantized cache Kq/Vq [n_kv][stride][hd] (bytes of
// format fmt: 1 int8, 2 E4M3) with row scales Ks/Vs [n_kv][stride]; below,
// kq / vq stand for the decoded byte values.  mode 1: softmax over q.(kq*ks)/sqrt(hd) of (vq*vs)
// in double.  mode 0: the device's rounding points: score =
// half((q.kq) * ks * 1/sqrt(hd)) with the dot in fp32, e = exp(s - m_part),
// P = half(e * vs) for the PV product while the partition sum adds the
// unrounded e, partitions merged like attention() above.
void attention_i8(const uint16_t* q, const int8_t* Kq, const float* Ks, const int8_t* Vq, const float* Vs,
                  uint16_t* out, int n_heads, int n_kv, int hd, int64_t stride, int T, int mode, int nparts,
                  int fmt = 1) {
  const int g = n_heads / n_kv;
  const float scale = 1.0f / std::sqrt((float)hd);
#pragma omp parallel for schedule(dynamic)
  for (int h = 0; h < n_heads; ++h) {
    const int kvh = h / g;
    const uint16_t* qh = q + (int64_t)h * hd;
    const int8_t* Kh = Kq + (int64_t)kvh * stride * hd;
    const int8_t* Vh = Vq + (int64_t)kvh * stride * hd;
    const float* ksh = Ks + (int64_t)kvh * stride;
    const float* vsh = Vs + (int64_t)kvh * stride;
    if (mode == 1) {
      std::vector<double> s(T);
      double mx = -INFINITY;
      for (int t = 0; t < T; ++t) {
        double a = 0.0;
        for (int d = 0; d < hd; ++d) a += (double)h2f(qh[d]) * ((double)kv_code(fmt, Kh[(int64_t)t * hd + d]) * ksh[t]);
        s[t] = a / std::sqrt((double)hd);
        mx = std::max(mx, s[t]);
      }
      double L = 0.0;
      std::vector<double> o(hd, 0.0);
      for (int t = 0; t < T; ++t) {
        const double e = std::exp(s[t] - mx);
        L += e;
        for (int d = 0; d < hd; ++d) o[d] += e * ((double)kv_code(fmt, Vh[(int64_t)t * hd + d]) * vsh[t]);
      }
      for (int d = 0; d < hd; ++d) out[(int64_t)h * hd + d] = f2h((float)(o[d] / L));
      continue;
    }
    const int chunk = (T + nparts - 1) / nparts;
    const int nonempty = (T + chunk - 1) / chunk;
    std::vector<float> pm(nonempty), ps(nonempty), po((size_t)nonempty * hd);
    for (int p = 0; p < nonempty; ++p) {
      const int t0 = p * chunk, t1 = std::min(t0 + chunk, T);
      std::vector<float> sc(t1 - t0);
      float mx = -1e30f;
      for (int t = t0; t < t1; ++t) {
        float a = 0.f;
        for (int d = 0; d < hd; ++d) a += h2f(qh[d]) * kv_code(fmt, Kh[(int64_t)t * hd + d]);
        sc[t - t0] = rh(a * ksh[t] * scale);
        mx = std::max(mx, sc[t - t0]);
      }
      float sum = 0.f;
      std::vector<float> pv(hd, 0.f);
      for (int t = t0; t < t1; ++t) {
        const float e = std::exp(sc[t - t0] - mx);
        sum += e;
        const float P = rh(e * vsh[t]);
        for (int d = 0; d < hd; ++d) pv[d] += P * kv_code(fmt, Vh[(int64_t)t * hd + d]);
      }
      pm[p] = mx;
      ps[p] = sum;
      for (int d = 0; d < hd; ++d) po[(size_t)p * hd + d] = pv[d];
    }
    float M = -1e30f;
    for (int p = 0; p < nonempty; ++p) M = std::max(M, pm[p]);
    std::vector<float> r(nonempty);
    float L = 0.f;
    for (int p = 0; p < nonempty; ++p) {
      r[p] = std::exp(pm[p] - M);
      L += ps[p] * r[p];
    }
    const float inv = 1.0f / (L + 1e-9f);
    for (int d = 0; d < hd; ++d) {
      float a = 0.f;
      for (int p = 0; p < nonempty; ++p) a += po[(size_t)p * hd + d] * r[p];
      out[(int64_t)h * hd + d] = f2h(a * inv);
    }
  }
}

// ---------------------------------------------------------------- argmax
// kernels.cu:907-961: order-preserving key, ties -> lowest index.
uint64_t argmax_key(float v, int idx) {
  uint32_t fu;
  std::memcpy(&fu, &v, 4);
  const uint32_t key = (fu & 0x80000000u) ? ~fu : (fu | 0x80000000u);
  return ((uint64_t)key << 32) | (uint32_t)(~idx);
}
int argmax(const uint16_t* logits, int vocab) {
  uint64_t best = 0;
  for (int i = 0; i < vocab; ++i) {
    const uint64_t k = argmax_key(h2f(logits[i]), i);
    if (k > best) best = k;
  }
  return (int)(~(uint32_t)(best & 0xffffffffu));
}

// kernels.cu:873-891 with each distinct id penalised once.
void penalty(uint16_t* logits, const int* hist, int n, int vocab, float pen) {
  std::vector<char> seen(vocab, 0);
  const float p = h2f(f2h(pen));
  for (int i = 0; i < n; ++i) {
    const int id = hist[i];
    if (id < 0 || id >= vocab || seen[id]) continue;
    seen[id] = 1;
    const float l = h2f(logits[id]);
    logits[id] = f2h(l < 0.f ? l * p : l / p);
  }
}

// ----------------------------------------------------------------- model
struct Cfg {
  int vocab, dim, inter, layers, heads, kv, hd, max_seq, quant, lm_fmt, tied;
};
struct Mat {
  std::vector<uint8_t> w;
  std::vector<uint16_t> s;
  int quant = 0;
  int64_t rows = 0, cols = 0;
};
struct Layer {
  std::vector<uint16_t> in_norm, post_norm, bq, bk, bv;
  Mat wq, wk, wv, wo, wg, wu, wd;
};
struct Model {
  Cfg c{};
  std::vector<uint16_t> embed, final_norm;
  Mat lm;      // lm.quant 0 fp16, 1 int8; empty when tied
  std::vector<Layer> L;
  int kv_slots = 0;
  std::vector<uint16_t> K, V;   // [layers][kv][kv_slots][hd]
  int kv8 = 0;                  // 0 fp16; 1 int8 / 2 E4M3 cache: Kq/Vq [layers][kv][kv_slots][hd] bytes, Ks/Vs [layers][kv][kv_slots]
  std::vector<int8_t> Kq, Vq;
  std::vector<float> Ks, Vs;
  std::vector<uint16_t> logits;
  int nparts = 64;
  double t_layers = 0.0, t_head = 0.0;   // seconds spent by the last forward() in the layers / after them
};

void gen_vec(std::vector<uint16_t>& v, int64_t n, uint64_t seed, int layer, int kind, float mean) {
  v.resize(n);
  const float mul = gen_mul(0.02);
  const uint64_t st = tensor_stream(layer, kind);
#pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) v[i] = gen_half(seed, st, (uint64_t)i, mul, mean);
}
void gen_mat(Mat& m, int64_t rows, int64_t cols, int quant, uint64_t seed, int layer, int kind) {
  std::vector<uint16_t> w;
  gen_vec(w, rows * cols, seed, layer, kind, 0.f);
  m.quant = quant;
  m.rows = rows;
  m.cols = cols;
  if (quant == 0) {
    m.w.resize(rows * cols * 2);
    std::memcpy(m.w.data(), w.data(), m.w.size());
    return;
  }
  m.w.assign(rows * row_bytes(quant, cols), 0);
  m.s.assign(rows * (cols / 128), 0);
  const int64_t rb = row_bytes(quant, cols);
#pragma omp parallel for
  for (int64_t r = 0; r < rows; ++r)
    quantize(quant, w.data() + r * cols, 1, cols, 128, m.w.data() + r * rb, m.s.data() + r * (cols / 128));
}

bool read_exact(FILE* f, void* p, size_t n) { return std::fread(p, 1, n, f) == n; }
bool read_vec(FILE* f, std::vector<uint16_t>& v, int64_t n) {
  v.resize(n);
  return read_exact(f, v.data(), n * 2);
}
bool read_mat(FILE* f, Mat& m, int64_t rows, int64_t cols, int quant) {
  m.quant = quant;
  m.rows = rows;
  m.cols = cols;
  m.w.resize(rows * row_bytes(quant, cols));
  if (!read_exact(f, m.w.data(), m.w.size())) return false;
  if (quant == 0) return true;
  m.s.resize(rows * (cols / 128));
  return read_exact(f, m.s.data(), m.s.size() * 2);
}

void alloc_kv(Model& m, int slots) {
  m.kv_slots = slots;
  const size_t n = (size_t)m.c.layers * m.c.kv * slots * m.c.hd;
  const size_t rows = (size_t)m.c.layers * m.c.kv * slots;
  if (m.kv8) {
    m.K.clear(); m.V.clear();
    m.Kq.assign(n, 0); m.Vq.assign(n, 0); m.Ks.assign(rows, 0.f); m.Vs.assign(rows, 0.f);
  } else {
    m.Kq.clear(); m.Vq.clear(); m.Ks.clear(); m.Vs.clear();
    m.K.assign(n, 0); m.V.assign(n, 0);
  }
  m.logits.assign(m.c.vocab, 0);
}

// Store one position's k (or v) rows of every kv head of layer l.
void store_kv(Model& m, int l, int pos, const uint16_t* k, const uint16_t* v) {
  const Cfg& c = m.c;
  for (int h = 0; h < c.kv; ++h) {
    const size_t row = ((size_t)l * c.kv + h) * m.kv_slots + pos;
    if (m.kv8) {
      quant_row_kv(m.kv8, k + h * c.hd, c.hd, m.Kq.data() + row * c.hd, m.Ks.data() + row);
      quant_row_kv(m.kv8, v + h * c.hd, c.hd, m.Vq.data() + row * c.hd, m.Vs.data() + row);
    } else {
      std::memcpy(m.K.data() + row * c.hd, k + h * c.hd, c.hd * 2);
      std::memcpy(m.V.data() + row * c.hd, v + h * c.hd, c.hd * 2);
    }
  }
}

// src/model.cu:76-181: one decode step; returns the argmax id.
int forward(Model& m, int token, int pos, const int* hist, int hlen, int mode) {
  const auto t0 = std::chrono::steady_clock::now();
  const Cfg& c = m.c;
  const int64_t d = c.dim, qd = (int64_t)c.heads * c.hd, kvd = (int64_t)c.kv * c.hd, I = c.inter;
  std::vector<uint16_t> x(m.embed.begin() + (int64_t)token * d, m.embed.begin() + (int64_t)(token + 1) * d);
  std::vector<uint16_t> xn(d), q(qd), k(kvd), v(kvd), att(qd), inter(I);
  const float eps = 1e-6f;
  auto gemv = [&](const Mat& W, const uint16_t* in, int64_t r) {
    return gemv_row(W.quant, W.w.data(), W.s.empty() ? nullptr : W.s.data(), in, r, W.cols, 128, mode);
  };
  for (int l = 0; l < c.layers; ++l) {
    Layer& Ly = m.L[l];
    rmsnorm(x.data(), Ly.in_norm.data(), xn.data(), d, eps, mode);
#pragma omp parallel for
    for (int64_t r = 0; r < qd; ++r) q[r] = f2h(gemv(Ly.wq, xn.data(), r) + h2f(Ly.bq[r]));
#pragma omp parallel for
    for (int64_t r = 0; r < kvd; ++r) {
      k[r] = f2h(gemv(Ly.wk, xn.data(), r) + h2f(Ly.bk[r]));
      v[r] = f2h(gemv(Ly.wv, xn.data(), r) + h2f(Ly.bv[r]));
    }
    rope(q.data(), c.heads, c.hd, pos, 1e6f);
    rope(k.data(), c.kv, c.hd, pos, 1e6f);
    const size_t lo = (size_t)l * c.kv * m.kv_slots * c.hd;
    store_kv(m, l, pos, k.data(), v.data());
    if (m.kv8) {
      const size_t ls = (size_t)l * c.kv * m.kv_slots;
      attention_i8(q.data(), m.Kq.data() + lo, m.Ks.data() + ls, m.Vq.data() + lo, m.Vs.data() + ls, att.data(),
                   c.heads, c.kv, c.hd, m.kv_slots, pos + 1, mode, m.nparts, m.kv8);
    } else {
      attention(q.data(), m.K.data() + lo, m.V.data() + lo, att.data(), c.heads, c.kv, c.hd, m.kv_slots, pos + 1,
                mode, m.nparts);
    }
#pragma omp parallel for
    for (int64_t r = 0; r < d; ++r) x[r] = f2h(h2f(x[r]) + gemv(Ly.wo, att.data(), r));   // kernels.cu:671
    rmsnorm(x.data(), Ly.post_norm.data(), xn.data(), d, eps, mode);
#pragma omp parallel for
    for (int64_t r = 0; r < I; ++r) {
      const float g = gemv(Ly.wg, xn.data(), r), u = gemv(Ly.wu, xn.data(), r);
      const float sig = 1.0f / (1.0f + std::exp(-g));   // kernels.cu:566
      inter[r] = f2h((g * sig) * u);
    }
#pragma omp parallel for
    for (int64_t r = 0; r < d; ++r) x[r] = f2h(h2f(x[r]) + gemv(Ly.wd, inter.data(), r));   // kernels.cu:621
  }
  const auto t1 = std::chrono::steady_clock::now();
  rmsnorm(x.data(), m.final_norm.data(), xn.data(), d, eps, mode);
  if (m.lm.rows) {
#pragma omp parallel for
    for (int64_t r = 0; r < c.vocab; ++r) m.logits[r] = f2h(gemv(m.lm, xn.data(), r));
  } else {   // tied: embed_tokens as an fp16 lm_head (kernels.cu:772-806)
#pragma omp parallel for
    for (int64_t r = 0; r < c.vocab; ++r)
      m.logits[r] = f2h(gemv_row(0, reinterpret_cast<const uint8_t*>(m.embed.data()), nullptr, xn.data(), r, d, 128, mode));
  }
  penalty(m.logits.data(), hist, hlen, c.vocab, 1.1f);
  const int id = argmax(m.logits.data(), c.vocab);
  const auto t2 = std::chrono::steady_clock::now();
  m.t_layers = std::chrono::duration<double>(t1 - t0).count();
  m.t_head = std::chrono::duration<double>(t2 - t1).count();
  return id;
}

}  // namespace

// ===================================================================== C API
extern "C" {

void or_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int or_max_threads(void) { return omp_get_max_threads(); }

uint16_t or_f2h(float f) { return f2h(f); }
float or_h2f(uint16_t h) { return h2f(h); }
uint16_t or_gen_half(uint64_t seed, uint64_t stream, uint64_t index, float sigma, float mean) {
  return gen_half(seed, stream, index, gen_mul(sigma), mean);
}
uint64_t or_tensor_stream(int layer, int kind) { return tensor_stream(layer, kind); }
uint64_t or_kv_stream(int layer, int kv_head, int kind) { return kv_stream(layer, kv_head, kind); }

void or_quantize(int quant, const uint16_t* w, int64_t rows, int64_t cols, int64_t group, uint8_t* q, uint16_t* s) {
  quantize(quant, w, rows, cols, group, q, s);
}

// y[r] (fp32, unrounded) for all rows; group 128 or 0 (per row).
void or_gemv(int quant, const uint8_t* W, const uint16_t* S, const uint16_t* x, float* y, int64_t rows, int64_t cols,
             int64_t group, int mode) {
#pragma omp parallel for
  for (int64_t r = 0; r < rows; ++r) y[r] = gemv_row(quant, W, S, x, r, cols, group, mode);
}
void or_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int64_t dim, float eps, int mode) {
  rmsnorm(x, w, out, dim, eps, mode);
}
void or_rope(uint16_t* v, int n_heads, int hd, int pos, float theta) { rope(v, n_heads, hd, pos, theta); }
void or_attention(const uint16_t* q, const uint16_t* K, const uint16_t* V, uint16_t* out, int n_heads, int n_kv,
                  int hd, int64_t stride, int T, int mode, int nparts) {
  attention(q, K, V, out, n_heads, n_kv, hd, stride, T, mode, nparts);
}
void or_quant_row_i8(const uint16_t* x, int n, int8_t* q, float* s) { quant_row_i8(x, n, q, s); }
void or_attention_i8(const uint16_t* q, const int8_t* Kq, const float* Ks, const int8_t* Vq, const float* Vs,
                     uint16_t* out, int n_heads, int n_kv, int hd, int64_t stride, int T, int mode, int nparts) {
  attention_i8(q, Kq, Ks, Vq, Vs, out, n_heads, n_kv, hd, stride, T, mode, nparts);
}
void or_attention_kvq(const uint16_t* q, const int8_t* Kq, const float* Ks, const int8_t* Vq, const float* Vs,
                      uint16_t* out, int n_heads, int n_kv, int hd, int64_t stride, int T, int mode, int nparts,
                      int fmt) {
  attention_i8(q, Kq, Ks, Vq, Vs, out, n_heads, n_kv, hd, stride, T, mode, nparts, fmt);
}
void or_quant_row_f8(const uint16_t* x, int n, uint8_t* q, float* s) { quant_row_f8(x, n, q, s); }
void or_e4m3_encode(const float* x, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = e4m3_encode(x[i]);
}
void or_e4m3_decode(const uint8_t* b, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = e4m3_decode(b[i]);
}
int or_argmax(const uint16_t* logits, int vocab) { return argmax(logits, vocab); }
void or_penalty(uint16_t* logits, const int* hist, int n, int vocab, float pen) { penalty(logits, hist, n, vocab, pen); }

// ---- model
void* or_model_synth(const int* cfg11, uint64_t seed, int kv_slots) {
  Model* m = new Model;
  Cfg& c = m->c;
  c.vocab = cfg11[0]; c.dim = cfg11[1]; c.inter = cfg11[2]; c.layers = cfg11[3]; c.heads = cfg11[4];
  c.kv = cfg11[5]; c.hd = cfg11[6]; c.max_seq = cfg11[7]; c.quant = cfg11[8]; c.lm_fmt = cfg11[9]; c.tied = cfg11[10];
  const int64_t d = c.dim, qd = (int64_t)c.heads * c.hd, kvd = (int64_t)c.kv * c.hd;
  gen_vec(m->embed, (int64_t)c.vocab * d, seed, -1, K_EMBED, 0.f);
  m->L.resize(c.layers);
  for (int l = 0; l < c.layers; ++l) {
    Layer& L = m->L[l];
    gen_vec(L.in_norm, d, seed, l, K_IN_NORM, 1.f);
    gen_mat(L.wq, qd, d, c.quant, seed, l, K_WQ);
    gen_vec(L.bq, qd, seed, l, K_BQ, 0.f);
    gen_mat(L.wk, kvd, d, c.quant, seed, l, K_WK);
    gen_vec(L.bk, kvd, seed, l, K_BK, 0.f);
    gen_mat(L.wv, kvd, d, c.quant, seed, l, K_WV);
    gen_vec(L.bv, kvd, seed, l, K_BV, 0.f);
    gen_mat(L.wo, d, qd, c.quant, seed, l, K_WO);
    gen_vec(L.post_norm, d, seed, l, K_POST_NORM, 1.f);
    gen_mat(L.wg, c.inter, d, c.quant, seed, l, K_WG);
    gen_mat(L.wu, c.inter, d, c.quant, seed, l, K_WU);
    gen_mat(L.wd, d, c.inter, c.quant, seed, l, K_WD);
  }
  gen_vec(m->final_norm, d, seed, -1, K_FINAL_NORM, 1.f);
  if (c.lm_fmt == 1) gen_mat(m->lm, c.vocab, d, 1, seed, -1, K_LM_HEAD);
  else if (!c.tied) gen_mat(m->lm, c.vocab, d, 0, seed, -1, K_LM_HEAD);
  alloc_kv(*m, kv_slots);
  return m;
}

// Independent reader of the export_weights.py layout (export_weights.py:267-323,
// load_weights.cpp:36-161).  Returns nullptr on any error.
void* or_model_load(const char* path, int kv_slots) {
  FILE* f = std::fopen(path, "rb");
  if (!f) return nullptr;
  int32_t h[11];
  if (std::fread(h, 4, 11, f) != 11 || h[0] != 0x5157454E) { std::fclose(f); return nullptr; }
  Model* m = new Model;
  Cfg& c = m->c;
  c.vocab = h[1]; c.dim = h[2]; c.inter = h[3]; c.layers = h[4]; c.heads = h[5]; c.kv = h[6]; c.hd = h[7];
  c.max_seq = h[8]; c.quant = h[9]; c.lm_fmt = h[10];
  std::fseek(f, 256, SEEK_SET);
  const int64_t d = c.dim, qd = (int64_t)c.heads * c.hd, kvd = (int64_t)c.kv * c.hd;
  bool ok = read_vec(f, m->embed, (int64_t)c.vocab * d);
  m->L.resize(c.layers);
  for (int l = 0; l < c.layers && ok; ++l) {
    Layer& L = m->L[l];
    ok = read_vec(f, L.in_norm, d) && read_mat(f, L.wq, qd, d, c.quant) && read_vec(f, L.bq, qd) &&
         read_mat(f, L.wk, kvd, d, c.quant) && read_vec(f, L.bk, kvd) && read_mat(f, L.wv, kvd, d, c.quant) &&
         read_vec(f, L.bv, kvd) && read_mat(f, L.wo, d, qd, c.quant) && read_vec(f, L.post_norm, d) &&
         read_mat(f, L.wg, c.inter, d, c.quant) && read_mat(f, L.wu, c.inter, d, c.quant) &&
         read_mat(f, L.wd, d, c.inter, c.quant);
  }
  ok = ok && read_vec(f, m->final_norm, d);
  c.tied = 0;
  if (ok && c.lm_fmt == 1) ok = read_mat(f, m->lm, c.vocab, d, 1);
  else if (ok) {
    const long cur = std::ftell(f);
    std::fseek(f, 0, SEEK_END);
    const long end = std::ftell(f);
    std::fseek(f, cur, SEEK_SET);
    if ((int64_t)(end - cur) >= (int64_t)c.vocab * d * 2) ok = read_mat(f, m->lm, c.vocab, d, 0);
    else c.tied = 1;
  }
  std::fclose(f);
  if (!ok) { delete m; return nullptr; }
  alloc_kv(*m, kv_slots);
  return m;
}

void or_model_free(void* h) { delete static_cast<Model*>(h); }
void or_model_set_nparts(void* h, int nparts) { static_cast<Model*>(h)->nparts = nparts; }

// KV slots [0, n_pos) of every layer from the generator (same values as the
// product's KV filler).
void or_model_fill_kv(void* h, int n_pos, uint64_t seed) {
  Model& m = *static_cast<Model*>(h);
  const float mul = gen_mul(1.0);
  const int hd = m.c.hd;
  for (int l = 0; l < m.c.layers; ++l)
    for (int kh = 0; kh < m.c.kv; ++kh) {
      const size_t row0 = ((size_t)l * m.c.kv + kh) * m.kv_slots;
#pragma omp parallel for
      for (int t = 0; t < n_pos; ++t) {
        std::vector<uint16_t> kr(hd), vr(hd);
        for (int d = 0; d < hd; ++d) {
          const uint64_t e = (uint64_t)t * hd + d;
          kr[d] = gen_half(seed, kv_stream(l, kh, 0), e, mul, 0.f);
          vr[d] = gen_half(seed, kv_stream(l, kh, 1), e, mul, 0.f);
        }
        const size_t row = row0 + t;
        if (m.kv8) {
          quant_row_kv(m.kv8, kr.data(), hd, m.Kq.data() + row * hd, m.Ks.data() + row);
          quant_row_kv(m.kv8, vr.data(), hd, m.Vq.data() + row * hd, m.Vs.data() + row);
        } else {
          std::memcpy(m.K.data() + row * hd, kr.data(), hd * 2);
          std::memcpy(m.V.data() + row * hd, vr.data(), hd * 2);
        }
      }
    }
}

// Switch the cache to fp16 (0), int8 (1) or E4M3 (2); clears it.
void or_model_set_kv8(void* h, int on) {
  Model& m = *static_cast<Model*>(h);
  m.kv8 = on;
  alloc_kv(m, m.kv_slots);
}

int or_model_forward(void* h, int token, int pos, const int* hist, int hlen, int mode) {
  Model& m = *static_cast<Model*>(h);
  if (pos < 0 || pos >= m.kv_slots || token < 0 || token >= m.c.vocab) return -1;
  return forward(m, token, pos, hist, hlen, mode);
}
// Wall time of the last forward(): [0] embedding + layers, [1] final norm +
// lm_head + penalty + argmax (for the CPU baseline's per-layer extrapolation).
void or_model_last_times(void* h, double* out) {
  const Model& m = *static_cast<Model*>(h);
  out[0] = m.t_layers;
  out[1] = m.t_head;
}
void or_model_logits(void* h, uint16_t* out) {
  Model& m = *static_cast<Model*>(h);
  std::memcpy(out, m.logits.data(), m.logits.size() * 2);
}
// Raw access for tests: kind 0/1 = K/V of (layer, kv_head) positions [0, n).
// (quantized cache: the dequantized value half(q * s) of each element.)
void or_model_kv(void* h, int layer, int kv_head, int kind, int n, uint16_t* out) {
  Model& m = *static_cast<Model*>(h);
  const size_t row0 = ((size_t)layer * m.c.kv + kv_head) * m.kv_slots;
  if (m.kv8) {
    const std::vector<int8_t>& Q = kind ? m.Vq : m.Kq;
    const std::vector<float>& S = kind ? m.Vs : m.Ks;
    for (int t = 0; t < n; ++t)
      for (int d = 0; d < m.c.hd; ++d)
        out[(size_t)t * m.c.hd + d] = f2h(kv_code(m.kv8, Q[(row0 + t) * m.c.hd + d]) * S[row0 + t]);
    return;
  }
  std::memcpy(out, (kind ? m.V : m.K).data() + row0 * m.c.hd, (size_t)n * m.c.hd * 2);
}
// Raw quantized rows (bytes) and scales (int8 / E4M3 cache only).
void or_model_kv8(void* h, int layer, int kv_head, int kind, int n, int8_t* q, float* sc) {
  Model& m = *static_cast<Model*>(h);
  const size_t row0 = ((size_t)layer * m.c.kv + kv_head) * m.kv_slots;
  std::memcpy(q, (kind ? m.Vq : m.Kq).data() + row0 * m.c.hd, (size_t)n * m.c.hd);
  std::memcpy(sc, (kind ? m.Vs : m.Ks).data() + row0, (size_t)n * 4);
}
// Copy one tensor out for op-level tests: kind = generator kind, which: 0
// weights/values, 1 scales.  Returns bytes copied (0 when absent).
int64_t or_model_tensor(void* h, int layer, int kind, int which, void* out) {
  Model& m = *static_cast<Model*>(h);
  const std::vector<uint16_t>* v = nullptr;
  const Mat* mt = nullptr;
  if (kind == K_EMBED) v = &m.embed;
  else if (kind == K_FINAL_NORM) v = &m.final_norm;
  else if (kind == K_LM_HEAD) mt = &m.lm;
  else {
    Layer& L = m.L[layer];
    switch (kind) {
      case K_IN_NORM: v = &L.in_norm; break;
      case K_POST_NORM: v = &L.post_norm; break;
      case K_BQ: v = &L.bq; break;
      case K_BK: v = &L.bk; break;
      case K_BV: v = &L.bv; break;
      case K_WQ: mt = &L.wq; break;
      case K_WK: mt = &L.wk; break;
      case K_WV: mt = &L.wv; break;
      case K_WO: mt = &L.wo; break;
      case K_WG: mt = &L.wg; break;
      case K_WU: mt = &L.wu; break;
      case K_WD: mt = &L.wd; break;
    }
  }
  if (v) {
    if (out) std::memcpy(out, v->data(), v->size() * 2);
    return (int64_t)v->size() * 2;
  }
  if (!mt) return 0;
  if (which == 0) {
    if (out) std::memcpy(out, mt->w.data(), mt->w.size());
    return (int64_t)mt->w.size();
  }
  if (out) std::memcpy(out, mt->s.data(), mt->s.size() * 2);
  return (int64_t)mt->s.size() * 2;
}

}  // extern "C"
