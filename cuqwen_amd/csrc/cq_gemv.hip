// GEMV kernels and their launcher (see cq_gemv.h for the design).
#include "cq_gemv.h"
#include "cq_internal.h"

#include <algorithm>

namespace cq {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kUnroll = 2;       // 16-byte chunks per lane in flight per row
constexpr int kMaxGemvBlocks = 2048;

template <int Q> __device__ __forceinline__ constexpr bool quantized() { return Q != CQ_QUANT_FP16; }

// Stage x (optionally RMS-normalised) into LDS as PLANES planes of 16-byte
// chunk slices, plus the per-chunk sum of x for the unpack bias.
template <int Q, bool NORM>
__device__ __forceinline__ void stage_x(const GemvArgs& a, u4_t* xs, float* sx, float* red) {
  using T = QTraits<Q>;
  const int K = a.K, NC = K / T::EPC;
  const _Float16* x = reinterpret_cast<const _Float16*>(a.x);
  const _Float16* nw = reinterpret_cast<const _Float16*>(a.norm_w);
  float inv = 1.f;
  if constexpr (NORM) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < K / 8; i += kBlock) {
      const h8_t v = __builtin_bit_cast(h8_t, load_u4(x + 8 * i));
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
    }
    ss = block_sum(ss, red);
    // eps travels as fp16 in the reference (kernels.cu:726, model.cu:96).
    inv = rsqrtf(ss / (float)K + (float)(_Float16)a.eps);
  }
  for (int c = threadIdx.x; c < NC; c += kBlock) {
    float s = 0.f;
#pragma unroll
    for (int p = 0; p < T::PLANES; ++p) {
      const int e0 = c * T::EPC + p * 8;
      const h8_t xv = __builtin_bit_cast(h8_t, load_u4(x + e0));
      float v[8];
      if constexpr (NORM) {
        const h8_t wv = __builtin_bit_cast(h8_t, load_u4(nw + e0));
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)(_Float16)(((float)xv[e] * inv) * (float)wv[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)xv[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[e];
      _Float16 o[8];
      plane_order<Q>(v, o);
      h8_t ov;
#pragma unroll
      for (int e = 0; e < 8; ++e) ov[e] = o[e];
      xs[p * NC + c] = __builtin_bit_cast(u4_t, ov);
    }
    if constexpr (quantized<Q>()) sx[c] = s;
  }
  __syncthreads();
}

// Rows handled by one wave unit.
template <int MODE, int R>
__device__ __forceinline__ int units_total(const GemvArgs& a) {
  if constexpr (MODE == GM_SWIGLU) return (a.N + R / 2 - 1) / (R / 2);
  else if constexpr (MODE == GM_QKV) return (a.n_heads + 2 * a.n_kv) * (a.head_dim / 2) / (R / 2);
  else return (a.N + R - 1) / R;
}

struct RowRef {
  int mat;    // matrix index into a.W / a.S / a.bias / a.out
  int row;    // row within that matrix
  bool valid;
};

template <int MODE, int R>
__device__ __forceinline__ RowRef row_of(const GemvArgs& a, int unit, int r) {
  RowRef rr;
  if constexpr (MODE == GM_SWIGLU) {
    const int o = unit * (R / 2) + (r % (R / 2));
    rr.mat = r < R / 2 ? 0 : 1;
    rr.valid = o < a.N;
    rr.row = rr.valid ? o : a.N - 1;
  } else if constexpr (MODE == GM_QKV) {
    constexpr int PP = R / 2;
    const int half = a.head_dim / 2;
    const int per_head = half / PP;
    const int h = unit / per_head;
    const int p = (unit % per_head) * PP + (r % PP);
    const int within = p + (r < PP ? 0 : half);
    int mh;
    if (h < a.n_heads) { rr.mat = 0; mh = h; }
    else if (h < a.n_heads + a.n_kv) { rr.mat = 1; mh = h - a.n_heads; }
    else { rr.mat = 2; mh = h - a.n_heads - a.n_kv; }
    rr.row = mh * a.head_dim + within;
    rr.valid = true;
  } else {
    const int row = unit * R + r;
    rr.mat = 0;
    rr.valid = row < a.N;
    rr.row = rr.valid ? row : a.N - 1;
  }
  return rr;
}

template <int R>
__device__ __forceinline__ float pick(const float (&acc)[R], int i) {
  float v = acc[0];
#pragma unroll
  for (int r = 1; r < R; ++r)
    if (i == r) v = acc[r];
  return v;
}

template <int Q, int MODE, int R, bool NORM, bool G128>
__global__ __launch_bounds__(kBlock) void gemv_kernel(const GemvArgs a) {
  using T = QTraits<Q>;
  extern __shared__ u4_t smem[];
  __shared__ float red[16];
  const int NC = a.K / T::EPC;
  u4_t* xs = smem;
  float* sx = reinterpret_cast<float*>(smem + T::PLANES * NC);

  stage_x<Q, NORM>(a, xs, sx, red);

  const int lane = threadIdx.x & (kWave - 1);
  const int n_units = units_total<MODE, R>(a);
  const int64_t rbytes = (int64_t)NC * 16;
  const int sstride = G128 ? a.K / kGroup : 1;

  for (int unit = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave; unit < n_units;
       unit += gridDim.x * kWavesPerBlock) {
    const char* rp[R];
    const _Float16* sp[R];
    RowRef rr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      rr[r] = row_of<MODE, R>(a, unit, r);
      rp[r] = reinterpret_cast<const char*>(a.W[rr[r].mat]) + (int64_t)rr[r].row * rbytes;
      if constexpr (quantized<Q>())
        sp[r] = reinterpret_cast<const _Float16*>(a.S[rr[r].mat]) + (int64_t)rr[r].row * sstride;
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;

    for (int base = 0; base < NC; base += kWave * kUnroll) {
      u4_t w[kUnroll][R];
      float sc[kUnroll][R];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int c = min(base + u * kWave + lane, NC - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          w[u][r] = load_u4_stream(rp[r] + (int64_t)c * 16);
          if constexpr (quantized<Q>()) sc[u][r] = (float)sp[r][G128 ? (c * T::EPC) / kGroup : 0];
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int c = base + u * kWave + lane;
        if (c < NC) {
          u4_t xv[T::PLANES];
#pragma unroll
          for (int p = 0; p < T::PLANES; ++p) xv[p] = xs[p * NC + c];
          if constexpr (quantized<Q>()) {
            const float corr = T::BIAS * sx[c];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = fmaf(sc[u][r], chunk_dot<Q>(w[u][r], xv) - corr, acc[r]);
          } else {
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] += chunk_dot<Q>(w[u][r], xv);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);

    // ------------------------------------------------------------ epilogue
    if constexpr (MODE == GM_STORE || MODE == GM_RESID) {
      if (lane < R) {
        const RowRef me = row_of<MODE, R>(a, unit, lane);
        if (me.valid) {
          float v = pick<R>(acc, lane);
          _Float16* out = reinterpret_cast<_Float16*>(a.out[0]);
          if constexpr (MODE == GM_RESID) {
            v = (float)out[me.row] + v;          // residual stays fp16 (kernels.cu:621, :671)
          } else if (a.bias[0]) {
            v += (float)reinterpret_cast<const _Float16*>(a.bias[0])[me.row];
          }
          _Float16 h = (_Float16)v;
          if (MODE == GM_STORE && a.stamp && a.stamp[me.row] == *a.d_epoch) {
            // repetition penalty on the fp16 logit (kernels.cu:885-888)
            const float pen = (float)(_Float16)a.penalty;
            const float l = (float)h;
            h = (_Float16)(l < 0.f ? l * pen : l / pen);
          }
          out[me.row] = h;
        }
      }
    } else if constexpr (MODE == GM_SWIGLU) {
      if (lane < R / 2) {
        const RowRef me = row_of<MODE, R>(a, unit, lane);
        if (me.valid) {
          const float g = pick<R>(acc, lane), u = pick<R>(acc, lane + R / 2);
          const float sig = 1.f / (1.f + expf(-g));    // kernels.cu:566
          reinterpret_cast<_Float16*>(a.out[0])[me.row] = (_Float16)((g * sig) * u);
        }
      }
    } else {  // GM_QKV: bias, RoPE on q/k, k/v into the cache
      constexpr int PP = R / 2;
      if (lane < PP) {
        const RowRef r0 = row_of<MODE, R>(a, unit, lane);
        const RowRef r1 = row_of<MODE, R>(a, unit, lane + PP);
        const _Float16* b = reinterpret_cast<const _Float16*>(a.bias[r0.mat]);
        float y0 = pick<R>(acc, lane), y1 = pick<R>(acc, lane + PP);
        if (b) { y0 += (float)b[r0.row]; y1 += (float)b[r1.row]; }
        y0 = (float)(_Float16)y0;            // q/k/v are fp16 before RoPE (kernels.cu:470)
        y1 = (float)(_Float16)y1;
        const int pos = *a.d_pos;
        const int hd = a.head_dim;
        const int i = r0.row % hd;           // rotation index in [0, hd/2)
        if (r0.mat < 2) {
          // NeoX rotation of (i, i + hd/2) (kernels.cu:370-398); the angle is
          // evaluated in double precision.
          const double freq = 1.0 / pow((double)a.rope_theta, (2.0 * i) / (double)hd);
          double sn, cs;
          sincos((double)pos * freq, &sn, &cs);
          const float c = (float)cs, s = (float)sn;
          const float o0 = add_rn(mul_rn(y0, c), -mul_rn(y1, s));
          const float o1 = add_rn(mul_rn(y1, c), mul_rn(y0, s));
          y0 = o0;
          y1 = o1;
        }
        const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1;
        _Float16* out = reinterpret_cast<_Float16*>(a.out[r0.mat]);
        if (out) { out[r0.row] = h0; out[r1.row] = h1; }
        if (r0.mat > 0 && a.kcache) {
          const int kvh = r0.row / hd, d0 = r0.row % hd, d1 = r1.row % hd;
          _Float16* cache = reinterpret_cast<_Float16*>(r0.mat == 1 ? a.kcache : a.vcache);
          if (r0.mat == 1) {
            cache[kv_k_offset(kvh, pos, d0, a.max_seq, hd)] = h0;
            cache[kv_k_offset(kvh, pos, d1, a.max_seq, hd)] = h1;
          } else {
            cache[kv_v_offset(kvh, pos, d0, a.max_seq, hd)] = h0;
            cache[kv_v_offset(kvh, pos, d1, a.max_seq, hd)] = h1;
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ host
static constexpr int rows_per_wave(int mode) {
  return mode == GM_STORE ? 4 : mode == GM_RESID ? 2 : mode == GM_SWIGLU ? 4 : 2;
}

int gemv_check(const GemvArgs& a) {
  if (a.quant < 0 || a.quant > 2) return fail(CQ_EINVAL, "gemv: bad quant type");
  if (a.K <= 0 || a.N <= 0) return fail(CQ_EINVAL, "gemv: empty shape");
  if (a.quant != CQ_QUANT_FP16 && a.K % kGroup) return fail(CQ_EINVAL, "gemv: cols must be a multiple of 128 for quantized weights");
  if (a.K % 8) return fail(CQ_EINVAL, "gemv: cols must be a multiple of 8");
  if (a.group != kGroup && a.group != 0) return fail(CQ_EINVAL, "gemv: group size must be 128 or 0 (per row)");
  if (!a.x || !a.W[0]) return fail(CQ_EINVAL, "gemv: null input");
  if (a.quant != CQ_QUANT_FP16 && !a.S[0]) return fail(CQ_EINVAL, "gemv: quantized weights need scales");
  if (a.mode == GM_SWIGLU && (!a.W[1] || (a.quant != CQ_QUANT_FP16 && !a.S[1])))
    return fail(CQ_EINVAL, "gemv: swiglu needs gate and up");
  if (a.mode == GM_QKV) {
    if (a.head_dim % 4 || a.head_dim > kMaxHeadDim || a.n_heads <= 0 || a.n_kv <= 0 || a.n_heads % a.n_kv)
      return fail(CQ_EINVAL, "gemv: bad head configuration");
    if (!a.W[1] || !a.W[2] || !a.d_pos) return fail(CQ_EINVAL, "gemv: qkv needs q, k, v weights and d_pos");
    if (a.kcache && a.max_seq % 32) return fail(CQ_EINVAL, "gemv: max_seq must be a multiple of 32");
  } else if (!a.out[0]) {
    return fail(CQ_EINVAL, "gemv: null output");
  }
  const int planes = a.quant == CQ_QUANT_INT4 ? 4 : a.quant == CQ_QUANT_INT8 ? 2 : 1;
  const int epc = a.quant == CQ_QUANT_INT4 ? 32 : a.quant == CQ_QUANT_INT8 ? 16 : 8;
  const size_t lds = (size_t)planes * (a.K / epc) * 16 + (a.quant ? (size_t)(a.K / epc) * 4 : 0);
  if (lds > 60 * 1024) return fail(CQ_EINVAL, "gemv: input vector too long for LDS staging");
  return CQ_OK;
}

template <int Q, int MODE, bool NORM, bool G128>
static int launch_t(const GemvArgs& a, hipStream_t stream) {
  using T = QTraits<Q>;
  constexpr int R = rows_per_wave(MODE);
  const int NC = a.K / T::EPC;
  const size_t lds = (size_t)T::PLANES * NC * 16 + (Q != CQ_QUANT_FP16 ? (size_t)NC * 4 : 0);
  int units;
  if (MODE == GM_SWIGLU) units = (a.N + R / 2 - 1) / (R / 2);
  else if (MODE == GM_QKV) units = (a.n_heads + 2 * a.n_kv) * (a.head_dim / 2) / (R / 2);
  else units = (a.N + R - 1) / R;
  const int blocks = std::min((units + kWavesPerBlock - 1) / kWavesPerBlock, kMaxGemvBlocks);
  hipLaunchKernelGGL((gemv_kernel<Q, MODE, R, NORM, G128>), dim3(blocks), dim3(kBlock), lds, stream, a);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

template <int Q, int MODE>
static int launch_q(const GemvArgs& a, hipStream_t stream) {
  const bool norm = a.norm_w != nullptr;
  if constexpr (MODE == GM_STORE) {
    if (a.group == 0) return norm ? launch_t<Q, MODE, true, false>(a, stream) : launch_t<Q, MODE, false, false>(a, stream);
    return norm ? launch_t<Q, MODE, true, true>(a, stream) : launch_t<Q, MODE, false, true>(a, stream);
  } else if constexpr (MODE == GM_RESID) {
    if (norm) return fail(CQ_EINVAL, "gemv: residual mode takes no norm");
    return launch_t<Q, MODE, false, true>(a, stream);
  } else {
    return norm ? launch_t<Q, MODE, true, true>(a, stream) : launch_t<Q, MODE, false, true>(a, stream);
  }
}

template <int Q>
static int launch_mode(const GemvArgs& a, hipStream_t stream) {
  switch (a.mode) {
    case GM_STORE: return launch_q<Q, GM_STORE>(a, stream);
    case GM_RESID: return launch_q<Q, GM_RESID>(a, stream);
    case GM_SWIGLU: return launch_q<Q, GM_SWIGLU>(a, stream);
    case GM_QKV: return launch_q<Q, GM_QKV>(a, stream);
  }
  return fail(CQ_EINVAL, "gemv: bad mode");
}

int launch_gemv(const GemvArgs& a, hipStream_t stream) {
  CQ_TRY(gemv_check(a));
  switch (a.quant) {
    case CQ_QUANT_FP16: return launch_mode<CQ_QUANT_FP16>(a, stream);
    case CQ_QUANT_INT8: return launch_mode<CQ_QUANT_INT8>(a, stream);
    default: return launch_mode<CQ_QUANT_INT4>(a, stream);
  }
}

// ------------------------------------------------------------- dequantize
// out[r][k] = q * scale through the same unpack helpers as the GEMV (test
// hook for the bit-exact unpack check).  One thread per 16-byte chunk.
template <int Q>
__global__ void dequant_kernel(const char* W, const _Float16* S, float* out, int rows, int cols, int group) {
  using T = QTraits<Q>;
  const int nc = cols / T::EPC;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)rows * nc) return;
  const int r = (int)(id / nc), c = (int)(id % nc);
  const u4_t w = load_u4(W + ((int64_t)r * nc + c) * 16);
  const float s = group ? (float)S[(int64_t)r * (cols / group) + (c * T::EPC) / group] : (float)S[r];
  float* o = out + (int64_t)r * cols + (int64_t)c * T::EPC;
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  if constexpr (Q == CQ_QUANT_INT4) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t f = words[p] ^ kInt4Flip;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const h2_t h = as_h2(int4_pair(f, i));
        o[8 * p + i] = ((float)h.x - kInt4Bias) * s;
        o[8 * p + i + 4] = ((float)h.y - kInt4Bias) * s;
      }
    }
  } else {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t f = words[p] ^ kInt8Flip;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const h2_t h = as_h2(int8_pair(f, i));
        o[4 * p + 2 * i] = ((float)h.x - kInt8Bias) * s;
        o[4 * p + 2 * i + 1] = ((float)h.y - kInt8Bias) * s;
      }
    }
  }
}

int launch_dequant(int quant, int group, const void* W, const __half* S, float* out, int rows, int cols,
                   hipStream_t stream) {
  if (quant != CQ_QUANT_INT8 && quant != CQ_QUANT_INT4) return fail(CQ_EINVAL, "dequant: quantized types only");
  if (cols % kGroup || rows <= 0 || (group != 0 && group != kGroup)) return fail(CQ_EINVAL, "dequant: bad shape");
  const int epc = quant == CQ_QUANT_INT4 ? 32 : 16;
  const int64_t n = (int64_t)rows * (cols / epc);
  const int blocks = (int)((n + 255) / 256);
  if (quant == CQ_QUANT_INT4)
    hipLaunchKernelGGL(dequant_kernel<CQ_QUANT_INT4>, dim3(blocks), dim3(256), 0, stream, (const char*)W,
                       (const _Float16*)S, out, rows, cols, group);
  else
    hipLaunchKernelGGL(dequant_kernel<CQ_QUANT_INT8>, dim3(blocks), dim3(256), 0, stream, (const char*)W,
                       (const _Float16*)S, out, rows, cols, group);
  CQ_HIP(hipGetLastError());
  return CQ_OK;
}

}  // namespace cq
