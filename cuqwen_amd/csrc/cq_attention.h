// Device building blocks of the FlashDecoding GQA attention (gfx950): the
// 32-key K/V tile of one wave, its loads, the online-softmax step with
// v_mfma_f32_16x16x32_f16, and the run-time partitioning of the context.
// Shared by the decode and prefill attention kernels.
#pragma once

#include "cq_device.h"
#include "cq_internal.h"

namespace cq {

constexpr int kAttnWaves = 8;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kAttnBlocksTarget = 256;   // one block per CU of MI355X
constexpr int kMinTilesPerPart = 1;      // short contexts spread over as many blocks as the slots allow
constexpr int kTileKeys = 32;

template <int HD>
struct KVTile {
  h8_t ka[2][HD / 32];
  h8_t va[HD / 16];
};

template <int HD>
__device__ __forceinline__ void load_tile(KVTile<HD>& t, const _Float16* kbase, const _Float16* vbase, int ti,
                                          int lane) {
  const _Float16* kt = kbase + (int64_t)ti * kTileKeys * HD;
  const _Float16* vt = vbase + (int64_t)ti * kTileKeys * HD;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int kk = 0; kk < HD / 32; ++kk)
      t.ka[st][kk] = __builtin_bit_cast(h8_t, load_u4_stream(kt + st * 16 * HD + (kk * 64 + lane) * 8));
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) t.va[dt] = __builtin_bit_cast(h8_t, load_u4_stream(vt + (dt * 64 + lane) * 8));
}

// The K and V of one kv head read through buffer resources.  A tile past
// the partition is read through a resource of zero records, which the
// buffer unit answers with zeros and no memory request: every path of the
// tile loop then issues the same loads, and the compiler's waits name
// exactly the tile being attended (a load issued only on some paths leaves
// it counting conservatively, i.e. waiting for the next tile's loads too).
// The tile offset is a scalar (soffset) and the lane's offset a loop
// invariant (voffset), so the loop writes no address registers.
struct KVRes {
  const _Float16* k;
  const _Float16* v;
  int bytes;   // one kv head's K (or V) slice
};

template <int HD>
__device__ __forceinline__ void load_tile(KVTile<HD>& t, const KVRes& r, int ti, bool valid, int lane) {
  constexpr int kNT = 2;   // cache policy: non-temporal (streamed once)
  const int n = valid ? r.bytes : 0;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(r.k), (short)0, n, kBufWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(r.v), (short)0, n, kBufWord3);
  const int soff = valid ? ti * (kTileKeys * HD * 2) : 0;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int kk = 0; kk < HD / 32; ++kk)
      t.ka[st][kk] = __builtin_bit_cast(
          h8_t, __builtin_amdgcn_raw_buffer_load_b128(rk, (st * 16 * HD + (kk * 64 + lane) * 8) * 2, soff, kNT));
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt)
    t.va[dt] = __builtin_bit_cast(h8_t, __builtin_amdgcn_raw_buffer_load_b128(rv, (dt * 64 + lane) * 8 * 2, soff, kNT));
}

// One 32-key tile of the online softmax for this wave.
template <int HD>
__device__ __forceinline__ void attend_tile(KVTile<HD>& t, const h8_t* qb, int ti, int T, float scale, int j,
                                            float& m, float& l, f4_t* o) {
  constexpr int KK = HD / 32, DT = HD / 16;
  f4_t s[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    s[st] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(t.ka[st][kk], qb[kk], s[st], 0, 0, 0);
  }
  // lane holds S^T[key = ti*32 + st*16 + 4j + i][head]
  const int key0 = ti * kTileKeys + 4 * j;
  const bool tail = (ti + 1) * kTileKeys > T;
  float sv[8];
  float mt = -INFINITY;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = (float)(_Float16)(s[st][i] * scale);
      if (tail && key0 + st * 16 + i >= T) v = -INFINITY;
      sv[st * 4 + i] = v;
      mt = fmaxf(mt, v);
    }
  mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
  mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
  const float mn = fmaxf(m, mt);
  const float alpha = __expf(m - mn);
  m = mn;
  l *= alpha;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
  h8_t pb;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = __expf(sv[e] - mn);
    l += p;
    pb[e] = (_Float16)p;
  }
  if (tail) {
    // keys past the end may hold anything; keep them out of P*V
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = ti * kTileKeys + (e < 4 ? 4 * j + e : 16 + 4 * j + e - 4);
        if (key >= T) t.va[dt][e] = (_Float16)0.f;
      }
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(t.va[dt], pb, o[dt], 0, 0, 0);
}

// All kernel arguments of a stage-1 launch in one batch of scalar loads
// (CQ_PIN); KV8 adds the quantized cache's.
template <bool KV8>
__device__ __forceinline__ void pin_attn_args(const AttnArgs& a) {
  CQ_PIN(gridDim.x); CQ_PIN(a.q); CQ_PIN(a.out); CQ_PIN(a.d_pos); CQ_PIN(a.n_heads); CQ_PIN(a.n_kv);
  CQ_PIN(a.max_seq); CQ_PIN(a.workspace);
  if constexpr (KV8) {
    CQ_PIN(a.kcache8); CQ_PIN(a.vcache8); CQ_PIN(a.kscale); CQ_PIN(a.vscale); CQ_PIN(a.k_new); CQ_PIN(a.v_new);
  } else {
    CQ_PIN(a.kcache); CQ_PIN(a.vcache);
  }
}

__device__ __forceinline__ int attn_nparts(int T, int P, int* tpp_out) {
  const int n_tiles = (T + kTileKeys - 1) / kTileKeys;
  int tpp = (n_tiles + P - 1) / P;
  if (tpp < kMinTilesPerPart) tpp = kMinTilesPerPart;
  *tpp_out = tpp;
  return (n_tiles + tpp - 1) / tpp;
}


// The wave's tiles ti, ti + 8, ... < tile1 of a partition, double-buffered:
// `A` already holds (or has in flight) tile ti; the next tile goes into the
// other buffer before the current one is computed.  On return m / l / o hold
// the wave's online-softmax state (l summed over the lane's 4 key slots).
template <int HD>
__device__ __forceinline__ void attend_partition(KVTile<HD>& A, KVTile<HD>& B, const h8_t* qb, int ti, int tile1,
                                                 int T, const KVRes& kv, int lane, float& m, float& l, f4_t* o) {
  const int j = lane >> 4;
  const float scale = 1.0f / sqrtf((float)HD);
  for (; ti < tile1; ti += 2 * kAttnWaves) {
    const int t1 = ti + kAttnWaves;
    load_tile<HD>(B, kv, t1, t1 < tile1, lane);
    attend_tile<HD>(A, qb, ti, T, scale, j, m, l, o);
    if (t1 >= tile1) break;
    load_tile<HD>(A, kv, t1 + kAttnWaves, t1 + kAttnWaves < tile1, lane);
    attend_tile<HD>(B, qb, t1, T, scale, j, m, l, o);
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
}

// Merge of the block's 8 waves in LDS (per wave m[16], l[16], O[16][HD]).
// The merged (m, l, O) of head hh goes to slot (kvh * 16 + hh) * Pmax + part
// of ws_m / ws_l / ws_o (O: HD floats per slot), or, when out is non-NULL
// (a single partition covers the context), the normalised output of the
// group's head hh to out[hh * HD + d] (global memory or LDS).
template <int HD>
__device__ __forceinline__ void block_merge_store(int kvh, int part, int g, float m, float l, const f4_t* o,
                                                  float* ws_m, float* ws_l, float* ws_o, int Pmax, _Float16* out) {
  constexpr int DT = HD / 16;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int h = lane & 15, j = lane >> 4;
  __shared__ float wm[kAttnWaves][16], wl[kAttnWaves][16];
  __shared__ float wo[kAttnWaves][16][HD + 1];
  if (j == 0) { wm[wave][h] = m; wl[wave][h] = l; }
  if (h < g) {   // the padding columns of the group are never read
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) wo[wave][h][dt * 16 + 4 * j + i] = o[dt][i];
  }
  __syncthreads();

  // One head per wave and round (HD is a multiple of 64, so the 64 items of
  // a wave share their head): lane w & 7 reads wave w's (m, l), the eight
  // rescale factors exp(m_w - M) are formed once per wave with 8-lane
  // reductions and broadcast through scalar registers, and each item is then
  // eight LDS reads and fused multiply-adds.
  const int w8 = lane & (kAttnWaves - 1);
  for (int idx = threadIdx.x; idx < g * HD; idx += kAttnThreads) {
    const int hh = __builtin_amdgcn_readfirstlane(idx / HD), d = idx % HD;
    const float mw = wm[w8][hh], lw = wl[w8][hh];
    float M = mw;
#pragma unroll
    for (int sh = 1; sh < kAttnWaves; sh <<= 1) M = fmaxf(M, __shfl_xor(M, sh, kWave));
    const float f = mw == -INFINITY ? 0.f : __expf(mw - M);
    float L = lw * f;
#pragma unroll
    for (int sh = 1; sh < kAttnWaves; sh <<= 1) L += __shfl_xor(L, sh, kWave);
    float O = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w)
      O = fmaf(wo[w][hh][d], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), w)), O);
    if (out) {
      out[hh * HD + d] = (_Float16)(O * (1.0f / (L + 1e-9f)));
    } else {
      const size_t slot = ((size_t)kvh * 16 + hh) * Pmax + part;
      ws_o[slot * HD + d] = O;
      if (d == 0) { ws_m[slot] = M; ws_l[slot] = L; }
    }
  }
}

// The engine's partials: workspace [m: n_kv*16*P][l: n_kv*16*P][o: n_kv*16*P*HD]
// floats, slots head-major so the merge reads each head's partitions as one
// contiguous run; a single partition writes the output itself.
template <int HD>
__device__ __forceinline__ void block_merge_write(const AttnArgs& a, int kvh, int part, int nparts, int g, float m,
                                                  float l, const f4_t* o) {
  float* ws_m = reinterpret_cast<float*>(a.workspace);
  const int Pmax = gridDim.x;
  float* ws_l = ws_m + (size_t)a.n_kv * Pmax * 16;
  float* ws_o = ws_l + (size_t)a.n_kv * Pmax * 16;
  block_merge_store<HD>(kvh, part, g, m, l, o, ws_m, ws_l, ws_o, Pmax,
                        nparts == 1 ? reinterpret_cast<_Float16*>(a.out) + (int64_t)kvh * g * HD : nullptr);
}

// ------------------------------------------------------- quantized KV cache
// One byte per element, int8 (CQ_KV_INT8) or OCP E4M3 (CQ_KV_FP8) codes.
// Same element layout as the fp16 cache (kv_k_offset / kv_v_offset count
// bytes instead of halves), so a lane's 8 elements of a matrix-core operand
// are 8 contiguous bytes; per-(position, kv head) fp32 scales live in
// separate [kv_head][max_seq] arrays.  The K scale multiplies the finished
// score, the V scale multiplies P before the PV product.
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

template <int HD>
struct KVTile8 {
  u2_t ka[2][HD / 32];
  u2_t va[HD / 16];
  f4_t ks[2], vs[2];   // scales of the lane's keys ti*32 + st*16 + 4j + i
};

__device__ __forceinline__ u2_t load_u2_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u2_t*>(p));
}

template <int HD>
__device__ __forceinline__ void load_tile8(KVTile8<HD>& t, const int8_t* kbase, const int8_t* vbase, const float* ksc,
                                           const float* vsc, int ti, int lane) {
  const int8_t* kt = kbase + (int64_t)ti * kTileKeys * HD;
  const int8_t* vt = vbase + (int64_t)ti * kTileKeys * HD;
  // one 16-byte load per lane fetches the operand pieces of two instructions
  // (kv8_k_offset / kv8_v_offset)
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk += 2) {
      const u4_t w = load_u4_stream(kt + st * 16 * HD + ((kk / 2) * 64 + lane) * 16);
      t.ka[st][kk] = u2_t{w.x, w.y};
      t.ka[st][kk + 1] = u2_t{w.z, w.w};
    }
#pragma unroll
  for (int dt = 0; dt < HD / 16; dt += 2) {
    const u4_t w = load_u4_stream(vt + ((dt / 2) * 64 + lane) * 16);
    t.va[dt] = u2_t{w.x, w.y};
    t.va[dt + 1] = u2_t{w.z, w.w};
  }
  const int j = lane >> 4;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    t.ks[st] = *reinterpret_cast<const f4_t*>(ksc + ti * kTileKeys + st * 16 + 4 * j);
    t.vs[st] = *reinterpret_cast<const f4_t*>(vsc + ti * kTileKeys + st * 16 + 4 * j);
  }
}

// The codes and scales of one kv head read through buffer resources, as
// KVRes does for the fp16 cache: a tile past the partition reads through
// resources of zero records (zeros, no memory request), so every path of
// the tile loop issues the same loads and each wait names only the tile
// being attended.
struct KVRes8 {
  const int8_t* k;
  const int8_t* v;
  const float* ks;
  const float* vs;
  int bytes;    // one kv head's K (or V) codes
  int sbytes;   // one kv head's K (or V) scales
};

template <int HD>
__device__ __forceinline__ void load_tile8(KVTile8<HD>& t, const KVRes8& r, int ti, bool valid, int lane) {
  constexpr int kNT = 2;   // cache policy: non-temporal (streamed once)
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(r.k), (short)0, valid ? r.bytes : 0, kBufWord3);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(r.v), (short)0, valid ? r.bytes : 0, kBufWord3);
  const __amdgpu_buffer_rsrc_t rks =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(r.ks), (short)0, valid ? r.sbytes : 0, kBufWord3);
  const __amdgpu_buffer_rsrc_t rvs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(r.vs), (short)0, valid ? r.sbytes : 0, kBufWord3);
  const int soff = valid ? ti * (kTileKeys * HD) : 0;
  const int ssoff = valid ? ti * (kTileKeys * 4) : 0;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk += 2) {
      const u4_t w = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, st * 16 * HD + ((kk / 2) * 64 + lane) * 16, soff, kNT));
      t.ka[st][kk] = u2_t{w.x, w.y};
      t.ka[st][kk + 1] = u2_t{w.z, w.w};
    }
#pragma unroll
  for (int dt = 0; dt < HD / 16; dt += 2) {
    const u4_t w =
        __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, ((dt / 2) * 64 + lane) * 16, soff, kNT));
    t.va[dt] = u2_t{w.x, w.y};
    t.va[dt + 1] = u2_t{w.z, w.w};
  }
  const int j = lane >> 4;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    t.ks[st] = __builtin_bit_cast(f4_t, __builtin_amdgcn_raw_buffer_load_b128(rks, (st * 16 + 4 * j) * 4, ssoff, 0));
    t.vs[st] = __builtin_bit_cast(f4_t, __builtin_amdgcn_raw_buffer_load_b128(rvs, (st * 16 + 4 * j) * 4, ssoff, 0));
  }
}

// 8 int8 (natural order) -> 8 exact fp16: (byte ^ 0x80) under the exponent
// pattern 0x64 is 1024 + q + 128; minus 1152 leaves q.
__device__ __forceinline__ h8_t i8x8_to_h8(u2_t w, uint32_t magic_v) {
  const uint32_t f0 = w.x ^ kInt8Flip, f1 = w.y ^ kInt8Flip;
  const h2_t bias = {(_Float16)-kInt8Bias, (_Float16)-kInt8Bias};
  u4_t o;
  o.x = as_u32(as_h2(int8_pair(f0, magic_v, 0)) + bias);
  o.y = as_u32(as_h2(int8_pair(f0, magic_v, 1)) + bias);
  o.z = as_u32(as_h2(int8_pair(f1, magic_v, 0)) + bias);
  o.w = as_u32(as_h2(int8_pair(f1, magic_v, 1)) + bias);
  return __builtin_bit_cast(h8_t, o);
}

// 8 E4M3 codes (natural order) -> 8 exact fp16 with the gfx950 converter
// (every E4M3 value is an fp16 value; the scale operand 1.0 leaves them).
__device__ __forceinline__ h8_t f8x8_to_h8(u2_t w) {
  u4_t o;
  o.x = as_u32(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.x, 1.0f, false));
  o.y = as_u32(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.x, 1.0f, true));
  o.z = as_u32(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.y, 1.0f, false));
  o.w = as_u32(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.y, 1.0f, true));
  return __builtin_bit_cast(h8_t, o);
}

// 8 codes of a quantized cache in format F (CQ_KV_INT8 / CQ_KV_FP8) as fp16.
template <int F>
__device__ __forceinline__ h8_t codes_to_h8(u2_t w, uint32_t magic_v) {
  if constexpr (F == CQ_KV_FP8) return f8x8_to_h8(w);
  else return i8x8_to_h8(w, magic_v);
}

// Largest code magnitude of a format (s = max|x| / it) and the code of one
// scaled element v = x / s: int8 rint clamped to +-127, E4M3 round to
// nearest even.
template <int F> __device__ __forceinline__ constexpr float kv_code_max() { return F == CQ_KV_FP8 ? 448.f : 127.f; }
template <int F>
__device__ __forceinline__ int8_t kv_encode(float v) {
  if constexpr (F == CQ_KV_FP8) return (int8_t)e4m3_bits(v);
  else return (int8_t)fminf(127.f, fmaxf(-127.f, rintf(v)));
}

// One 32-key tile of the online softmax over a one-byte cache (F: int8 codes
// or FP8 E4M3 codes).  Keys at or past t_lane (this lane's column limit) are
// masked; P of masked keys is exactly 0 (the encoders never write a NaN code,
// stale scales are selected out).  Rounding as the fp16 path:
// score = half(s * k_scale * 1/sqrt(hd)), P = half(p * v_scale) for the
// product, the row sum over the unrounded p.
template <int HD, int F = CQ_KV_INT8>
__device__ __forceinline__ void attend_tile8(KVTile8<HD>& t, const h8_t* qb, int ti, int t_lane, float scale, int j,
                                             float& m, float& l, f4_t* o, uint32_t magic_v) {
  constexpr int KK = HD / 32, DT = HD / 16;
  f4_t s[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    s[st] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_h8<F>(t.ka[st][kk], magic_v), qb[kk], s[st], 0, 0, 0);
  }
  const int key0 = ti * kTileKeys + 4 * j;
  float sv[8];
  float mt = -INFINITY;
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = (float)(_Float16)(s[st][i] * t.ks[st][i] * scale);
      if (key0 + st * 16 + i >= t_lane) v = -INFINITY;
      sv[st * 4 + i] = v;
      mt = fmaxf(mt, v);
    }
  mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
  mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
  const float mn = fmaxf(m, mt);
  const float alpha = m == -INFINITY ? 0.f : __expf(m - mn);
  m = mn;
  l *= alpha;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
  h8_t pb;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = sv[e] == -INFINITY ? 0.f : __expf(sv[e] - mn);
    l += p;
    pb[e] = sv[e] == -INFINITY ? (_Float16)0.f : (_Float16)(p * t.vs[e >> 2][e & 3]);
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_h8<F>(t.va[dt], magic_v), pb, o[dt], 0, 0, 0);
}

// Per-row quantization in format F (s = max|x| / code max, q = code of
// x / s, a zero row keeps s = 0 and q = 0) of the HD-element row x held by
// one wave (HD / 64 consecutive elements per lane); returns s, writes
// q[0..HD/64).
template <int HD, int F>
__device__ __forceinline__ float quant_row8_wave(const float* x, int8_t* q) {
  constexpr int E = HD / kWave;
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = wave_max(amax);
  const float s = amax / kv_code_max<F>();
#pragma unroll
  for (int i = 0; i < E; ++i) q[i] = s == 0.f ? (int8_t)0 : kv_encode<F>(x[i] / s);
  return s;
}

// Replaces key kp (0..31) of a loaded tile by the new row (kq / vq: HD int8
// each in LDS, scales ksn / vsn).
template <int HD>
__device__ __forceinline__ void patch_key8(KVTile8<HD>& t, int kp, const int8_t* kq, const int8_t* vq, float ksn,
                                           float vsn, int lane) {
  // register indices stay compile-time (unrolled, selected by compares), so
  // the tile never leaves the register file
  const int kst = kp >> 4, r = kp & 15, j = lane >> 4;
  const bool krow = (lane & 15) == r, vslot = j == (r >> 2);
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    if (st != kst) continue;
    if (krow) {
#pragma unroll
      for (int kk = 0; kk < HD / 32; ++kk) t.ka[st][kk] = *reinterpret_cast<const u2_t*>(kq + kk * 32 + j * 8);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!vslot || i != (r & 3)) continue;
      t.ks[st][i] = ksn;
      t.vs[st][i] = vsn;
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) {
        const uint32_t b = (uint8_t)vq[dt * 16 + (lane & 15)];
        const int e = st * 4 + i, sh = (e & 3) * 8;
        if (e < 4) t.va[dt].x = (t.va[dt].x & ~(0xFFu << sh)) | (b << sh);
        else t.va[dt].y = (t.va[dt].y & ~(0xFFu << sh)) | (b << sh);
      }
    }
  }
}

}  // namespace cq
