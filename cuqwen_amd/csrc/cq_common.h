// Shared host/device definitions of the MI355X decode engine: status
// handling, the synthetic data generator, quantization constants and the KV
// cache tile layout.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include <cstddef>
#include <string>

#include "../../include/cuqwen.h"

#define CQ_HD __host__ __device__ __forceinline__

// ---------------------------------------------------------------- errors
namespace cq {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
}  // namespace cq

#define CQ_HIP(call)                                                                     \
  do {                                                                                   \
    hipError_t e_ = (call);                                                              \
    if (e_ != hipSuccess)                                                                \
      return cq::fail(CQ_EHIP, std::string(#call) + ": " + hipGetErrorString(e_) +       \
                                   " at " + __FILE__ + ":" + std::to_string(__LINE__)); \
  } while (0)

#define CQ_TRY(call)          \
  do {                        \
    int r_ = (call);          \
    if (r_ != CQ_OK) return r_; \
  } while (0)

namespace cq {

// ------------------------------------------------------- fp16 bit helpers
CQ_HD uint32_t float_bits(float f) {
#ifdef __HIP_DEVICE_COMPILE__
  return __float_as_uint(f);
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
#endif
}
CQ_HD float bits_float(uint32_t u) {
#ifdef __HIP_DEVICE_COMPILE__
  return __uint_as_float(u);
#else
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
#endif
}
// float -> IEEE binary16, round to nearest even, in integer arithmetic only,
// so the generator and the quantizer give the same bits on host and device
// whatever the hardware's fp16 denormal mode.
CQ_HD uint16_t f2h_bits(float f) {
  const uint32_t x = float_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
  if (ax >= 0x477FF000u) return sign | 0x7C00u;            // rounds to >= 65520: inf
  if (ax >= 0x38800000u) {                                 // normal fp16
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  if (ax <= 0x33000000u) return sign;                      // <= 2^-25: rounds to zero
  const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
  const uint32_t shift = 126u - e;                         // 14..24: units of 2^-24
  uint32_t q = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return (uint16_t)(sign | q);
}
CQ_HD float h2f_bits(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// ------------------------------------------------------- E4M3 (OCP fp8)
// Codes of the fp8 KV cache: sign, 4 exponent bits (bias 7), 3 mantissa
// bits, subnormals m * 2^-9, largest finite 448 (0x7E); no infinities.
// Finite v to E4M3 with round to nearest, ties to an even mantissa, values
// past 448 saturating (the quantizer never produces them: |x / s| <= 448),
// in integer arithmetic so host and device give the same code.
CQ_HD uint8_t e4m3_bits(float v) {
  const uint32_t x = float_bits(v);
  const uint8_t sign = (uint8_t)((x >> 24) & 0x80u);
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x43E80000u) return sign | 0x7Eu;   // >= 464, the 448 / 480 midpoint (ties to 448, even)
  if (ax < 0x3C800000u) {                        // below 2^-6: the subnormal grid, units of 2^-9
    if (ax < 0x3A800000u) return sign;           // at most 2^-10 (the tie with 0 goes to 0)
    const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 141u - e;             // value / 2^-9 = m * 2^(e - 141): shift 21..24
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint8_t)(sign | q);                  // q = 8 is 2^-6, code 0x08
  }
  uint32_t code = ((((ax >> 23) - 120u)) << 3) | ((ax >> 20) & 7u);   // exponent - 127 + 7
  const uint32_t rem = ax & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (code & 1u))) ++code;   // a carry moves to the next binade
  return (uint8_t)(sign | (code > 0x7Eu ? 0x7Eu : code));
}
// Value of a finite E4M3 code.
CQ_HD float e4m3_value(uint8_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  const float a = e == 0 ? (float)m * 0.001953125f : bits_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -a : a;
}

// -------------------------------------------------- synthetic generator
// splitmix64 finaliser (Steele, Lea, Flood 2014).
CQ_HD uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
CQ_HD uint64_t rand64(uint64_t seed, uint64_t stream, uint64_t index) {
  uint64_t key = mix64(seed + 0x9E3779B97F4A7C15ull * (stream + 1));
  return mix64(key + 0x9E3779B97F4A7C15ull * (index + 1));
}
// Irwin-Hall sum of four 16-bit uniforms: mean 131070, sd 37836.5 (var =
// 4 * (65536^2 - 1) / 12).  The centred sum is an exact integer below 2^24,
// so one fp32 multiply by `mul` (sigma / sd, computed once on the host) and
// one round-to-nearest-even to fp16 give bit-identical results anywhere.
constexpr double kIrwinHallSd = 37836.51;
CQ_HD int32_t irwin_hall_centred(uint64_t r) {
  int32_t s = (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) +
              (int32_t)((r >> 32) & 0xFFFF) + (int32_t)((r >> 48) & 0xFFFF);
  return s - 131070;
}
// Separately rounded multiply and add: the device compiler would otherwise
// contract them into one fma and differ from the host by an ulp.
CQ_HD float mul_rn(float a, float b) {
#ifdef __HIP_DEVICE_COMPILE__
  return __fmul_rn(a, b);
#else
  return a * b;
#endif
}
CQ_HD float add_rn(float a, float b) {
#ifdef __HIP_DEVICE_COMPILE__
  return __fadd_rn(a, b);
#else
  return a + b;
#endif
}
CQ_HD float synth_value_f32(uint64_t seed, uint64_t stream, uint64_t index, float mul, float mean) {
  return add_rn(mul_rn((float)irwin_hall_centred(rand64(seed, stream, index)), mul), mean);
}
CQ_HD uint16_t synth_half(uint64_t seed, uint64_t stream, uint64_t index, float mul, float mean) {
  return f2h_bits(synth_value_f32(seed, stream, index, mul, mean));
}
inline float synth_mul(double sigma) { return (float)(sigma / kIrwinHallSd); }

// Tensor kinds of the generator's stream ids (layer * 32 + kind).
enum TensorKind {
  TK_EMBED = 0, TK_FINAL_NORM = 1, TK_LM_HEAD = 2,
  TK_IN_NORM = 3, TK_WQ = 4, TK_BQ = 5, TK_WK = 6, TK_BK = 7, TK_WV = 8, TK_BV = 9,
  TK_WO = 10, TK_POST_NORM = 11, TK_WG = 12, TK_WU = 13, TK_WD = 14
};
CQ_HD uint64_t tensor_stream(int layer, int kind) { return (uint64_t)(layer + 1) * 32u + (uint64_t)kind; }
CQ_HD uint64_t kv_stream(int layer, int kv_head, int kind) {
  return 0x100000000ull + ((uint64_t)layer * 4096u + (uint64_t)kv_head) * 2u + (uint64_t)kind;
}
// Distribution of each synthetic tensor: N(0, 0.02) weights and biases,
// norm weights N(1, 0.02) (N(0, 0.02) norm weights would zero the residual).
constexpr double kWeightSigma = 0.02;

// ------------------------------------------------------------ quantization
constexpr int kGroup = 128;
constexpr int kMaxHeadDim = 128;

// ----------------------------------------------------------- KV cache tiles
// Per (layer, kv head) the cache holds max_seq_len slots.  K is stored in
// 16-key tiles in the A-operand order of v_mfma_f32_16x16x32_f16 with keys as
// rows: element (t, d) with d = kk*32 + j*8 + e sits at
// tile(t/16) + ((kk*64 + j*16 + t%16) * 8 + e).  V is stored in 32-key tiles
// in the A-operand order of O^T = V^T P^T: element (t, d) with
// d = dt*16 + dl and t%32 -> (j, e) sits at tile(t/32) + ((dt*64 + j*16 + dl)*8 + e)
// where key slot j*8+e holds key 4j+e (e<4) or 16+4j+(e-4) (e>=4), the order
// in which the S^T accumulator tiles hand keys to each lane.
CQ_HD int64_t kv_k_offset(int kv_head, int t, int d, int max_seq, int hd) {
  const int kk = d >> 5, j = (d >> 3) & 3, e = d & 7;
  const int64_t tile = (int64_t)(t >> 4) * 16 * hd;
  return (int64_t)kv_head * max_seq * hd + tile + ((kk * 64 + j * 16 + (t & 15)) * 8 + e);
}
CQ_HD int64_t kv_v_offset(int kv_head, int t, int d, int max_seq, int hd) {
  const int dt = d >> 4, dl = d & 15;
  const int t32 = t & 31;
  const int j = (t32 & 15) >> 2;
  const int e = (t32 & 3) + ((t32 >> 4) << 2);
  const int64_t tile = (int64_t)(t >> 5) * 32 * hd;
  return (int64_t)kv_head * max_seq * hd + tile + ((dt * 64 + j * 16 + dl) * 8 + e);
}

// The int8 / E4M3 caches (one byte per element) keep the same tiles and
// operand order, with the 8-byte operand pieces of instruction pairs
// (kk, kk+1) for K and (dt, dt+1) for V placed side by side, so one 16-byte
// load per lane fetches two operands: piece (i, lane) of the fp16 layout
// (i = kk or dt) sits at ((i/2)*64 + lane)*16 + (i%2)*8.
CQ_HD int64_t kv8_k_offset(int kv_head, int t, int d, int max_seq, int hd) {
  const int kk = d >> 5, j = (d >> 3) & 3, e = d & 7;
  const int64_t tile = (int64_t)(t >> 4) * 16 * hd;
  return (int64_t)kv_head * max_seq * hd + tile + (((kk >> 1) * 64 + j * 16 + (t & 15)) * 16 + (kk & 1) * 8 + e);
}
CQ_HD int64_t kv8_v_offset(int kv_head, int t, int d, int max_seq, int hd) {
  const int dt = d >> 4, dl = d & 15;
  const int t32 = t & 31;
  const int j = (t32 & 15) >> 2;
  const int e = (t32 & 3) + ((t32 >> 4) << 2);
  const int64_t tile = (int64_t)(t >> 5) * 32 * hd;
  return (int64_t)kv_head * max_seq * hd + tile + (((dt >> 1) * 64 + j * 16 + dl) * 16 + (dt & 1) * 8 + e);
}

// Weight row bytes for `cols` logical weights (include/config.h:36-40).
inline int64_t row_bytes(int quant, int64_t cols) {
  return quant == CQ_QUANT_INT4 ? cols / 2 : quant == CQ_QUANT_INT8 ? cols : cols * 2;
}

}  // namespace cq
