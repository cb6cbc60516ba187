// mla_kernels.hip — gfx950 kernels for the MLA latent-KV-cache hot path.
//
//   mla_append_*      fused kv_norm LayerNorm + RoPE(k_pe) + optional e4m3
//                     quantisation + scatter into the ragged cache
//                     (reference: models/mla.py:307-323, :409-414)
//   mla_decode_mfma   absorbed attention over the latent cache, bf16 MFMA,
//                     split-KV partials (reference: models/mla.py:417-487)
//   mla_decode_f32    the same maths in fp32 on the VALU, for fp32 models
//   mla_merge_kernel  log-sum-exp merge of split-KV partials
//
// Geometry is fixed at R = 256 (kv_lora_rank), P = 64 (rope dim), H = 16.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mla_args.h"
#include "numerics.h"

namespace swamla {

constexpr int kR = 256;
constexpr int kP = 64;
constexpr int kH = 16;
constexpr int kKC = kR + kP;  // 320 channels scored per cached token

// ---------------------------------------------------------------------------
// Split plan (shared by decode and merge; mirrored by mla_split_count).
// ---------------------------------------------------------------------------
SW_HD int split_chunk(int L, int n_splits, int min_chunk) {
  int c = (L + n_splits - 1) / n_splits;
  if (c < min_chunk) c = min_chunk;
  return (c + 63) & ~63;
}
SW_HD int split_count(int L, int n_splits, int min_chunk) {
  if (L <= 0) return 0;
  int c = split_chunk(L, n_splits, min_chunk);
  return (L + c - 1) / c;
}

// ---------------------------------------------------------------------------
// Small helpers
// ---------------------------------------------------------------------------
template <int DT>
struct Elem;
template <>
struct Elem<0> {  // fp32
  using T = float;
  static __device__ __forceinline__ float ld(const T* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ T from_f32(float f) { return f; }
  static __device__ __forceinline__ T from_f64(double d) { return static_cast<float>(d); }
  // op-by-op rounding of eager fp32 math: contraction into a fused
  // multiply-add is switched off (HIP's __fmul_rn is a plain multiply that
  // the compiler may otherwise fuse with the following add).
  static __device__ __forceinline__ float mul(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
  }
  static __device__ __forceinline__ float add(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
  }
  static __device__ __forceinline__ float sub(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
  }
};
template <>
struct Elem<1> {  // bf16
  using T = uint16_t;
  static __device__ __forceinline__ float ld(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ T from_f32(float f) { return f32_to_bf16(f); }
  static __device__ __forceinline__ T from_f64(double d) { return f64_to_bf16(d); }
  // eager bf16 math: compute in fp32, round to bf16 after every op
  static __device__ __forceinline__ float mul(float a, float b) {
#pragma clang fp contract(off)
    return round_bf16(a * b);
  }
  static __device__ __forceinline__ float add(float a, float b) {
#pragma clang fp contract(off)
    return round_bf16(a + b);
  }
  static __device__ __forceinline__ float sub(float a, float b) {
#pragma clang fp contract(off)
    return round_bf16(a - b);
  }
};

// Interleaved-pair RoPE of one pair (positional_encoding.py:37-41, :57-60):
// o1 = x1*c - x2*s, o2 = x2*c + x1*s, rounded after every op in the model dtype.
template <int DT>
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float& o1,
                                          float& o2) {
  using E = Elem<DT>;
  o1 = E::sub(E::mul(x1, c), E::mul(x2, s));
  o2 = E::add(E::mul(x2, c), E::mul(x1, s));
}

__device__ __forceinline__ double shfl_xor_f64(double v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ float shfl_xor_f32(float v, int m) { return __shfl_xor(v, m, 64); }

// ---------------------------------------------------------------------------
// Kernel 1: fused append.  One wavefront per token, 4 tokens per block.
// ---------------------------------------------------------------------------

// IN_DT: 0 fp32 / 1 bf16 (model dtype; also k_pe cache dtype).
// C_DT : 0 fp32 / 1 bf16 / 2 e4m3 (latent cache dtype).
template <int IN_DT, int C_DT>
__global__ __launch_bounds__(256) void mla_append_kernel(AppendArgs a) {
  // Every multiply / add below is rounded on its own: the LayerNorm must
  // reproduce the fixed-order fp64 statement exactly.
#pragma clang fp contract(off)
  using E = Elem<IN_DT>;
  using T = typename E::T;
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= a.n_tok) return;
  const int b = a.seq_idx[tok], pos = a.dst_pos[tok], rp = a.rope_pos[tok];
  if (b < 0 || b >= a.cache_b || pos < 0 || pos >= a.cache_s || rp < 0 || rp >= a.rope_len) {
    if (lane == 0 && a.err_flag) a.err_flag[0] = 1;
    return;
  }
  const T* row = static_cast<const T*>(a.kv_in) + static_cast<int64_t>(tok) * a.in_rs;
  const T* w = static_cast<const T*>(a.ln_w);
  const T* bb = static_cast<const T*>(a.ln_b);

  // --- LayerNorm over c[0..255]: lane owns channels 4*lane .. 4*lane+3.
  // Statistics in fp64; fixed order: in-lane left-to-right, then xor
  // butterfly 1,2,4,...,32 (every lane ends with the same total).
  double x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = static_cast<double>(E::ld(row, 4 * lane + i));
  double s = ((x[0] + x[1]) + x[2]) + x[3];
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) s = s + shfl_xor_f64(s, m);
  const double mean = s * (1.0 / 256.0);
  double d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = x[i] - mean;
  double q = ((d[0] * d[0] + d[1] * d[1]) + d[2] * d[2]) + d[3] * d[3];
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) q = q + shfl_xor_f64(q, m);
  const double var = q * (1.0 / 256.0);
  // correctly rounded square root and IEEE division
  const double rstd = 1.0 / __dsqrt_rn(var + static_cast<double>(a.eps));
  double y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const double wi = static_cast<double>(E::ld(w, 4 * lane + i));
    const double bi = static_cast<double>(E::ld(bb, 4 * lane + i));
    y[i] = (d[i] * rstd) * wi + bi;
  }

  const int64_t crow = static_cast<int64_t>(b) * a.cache_s + pos;
  if constexpr (C_DT == 0) {
    float4 o = make_float4(static_cast<float>(y[0]), static_cast<float>(y[1]),
                           static_cast<float>(y[2]), static_cast<float>(y[3]));
    reinterpret_cast<float4*>(static_cast<float*>(a.ckv) + crow * kR)[lane] = o;
  } else if constexpr (C_DT == 1) {
    uint2 o;
    o.x = f64_to_bf16(y[0]) | (static_cast<uint32_t>(f64_to_bf16(y[1])) << 16);
    o.y = f64_to_bf16(y[2]) | (static_cast<uint32_t>(f64_to_bf16(y[3])) << 16);
    reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.ckv) + crow * kR)[lane] = o;
  } else {
    // e4m3 per-token: y is first rounded to bf16 (the value a bf16 cache
    // would hold), amax over the token, scale = max(amax,1e-12)/448.
    float yb[4];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      yb[i] = bf16_to_f32(f64_to_bf16(y[i]));
      amax = fmaxf(amax, fabsf(yb[i]));
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) amax = fmaxf(amax, shfl_xor_f32(amax, m));
    const float scale = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
    uint32_t codes = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      codes |= static_cast<uint32_t>(f32_to_e4m3(__fdiv_rn(yb[i], scale))) << (8 * i);
    reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.ckv) + crow * kR)[lane] = codes;
    if (lane == 0) a.ckv_scale[crow] = scale;
  }

  // --- RoPE on k_pe: lanes 0..31 own pair i = lane.
  if (lane < kP / 2) {
    const T* ct = static_cast<const T*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
    const T* st = static_cast<const T*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
    const float x1 = E::ld(row, kR + 2 * lane), x2 = E::ld(row, kR + 2 * lane + 1);
    float o1, o2;
    rope_pair<IN_DT>(x1, x2, E::ld(ct, lane), E::ld(st, lane), o1, o2);
    T* dst = static_cast<T*>(a.kpe) + crow * kP + 2 * lane;
    dst[0] = E::from_f32(o1);
    dst[1] = E::from_f32(o2);
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: absorbed decode attention, bf16 MFMA (cache bf16 or e4m3).
//
// Block = 4 wavefronts, one block per (query row, split).  Wave w owns the
// 16-token sub-tiles base = t0 + 16*w + 64*i.  Per sub-tile:
//   S^T[16 tok x 16 heads] = K[16 tok x 320] . Q^T[320 x 16 heads]
//       10 x mfma_f32_16x16x32_bf16, K operand straight from 16 B global loads
//   online softmax per head (lane-local: a lane owns head l%16, tokens 4g..4g+3)
//   O^T[256 ch x 16 heads] += C^T[256 x 16 tok] . P^T[16 tok x 16 heads]
//       16 x mfma_f32_16x16x16_bf16; C^T is read from a wave-private LDS
//       tile written transposed from the same registers that fed S.
// The four waves' (m, l, O) are merged through LDS at the end.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));


constexpr int kSub = 16;             // tokens per wave sub-tile
constexpr int kWaves = 4;
constexpr int kTStride = 20;         // bf16 elements per transposed-tile row (16 + pad)
constexpr int kTileElems = kR * kTStride;
constexpr int kOStride = kR + 4;     // fp32 row stride of the cross-wave merge buffer
static_assert(kH * kOStride * 4 <= kWaves * kTileElems * 2, "merge buffer must fit the tiles");
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// Channel order of the K dimension for MFMA step s (0..9) and lane group g:
// the 8 channels [chan(s,g), +8).  bf16 cache: plain order.  e4m3 cache: a
// 16 B load of 16 codes feeds steps 2j and 2j+1, so channels interleave.
template <int C_DT>
__device__ __forceinline__ int chan_of(int s, int g) {
  if constexpr (C_DT == 2) return 64 * (s >> 1) + 16 * g + 8 * (s & 1);
  return 32 * s + 8 * g;
}

template <int C_DT>
__global__ __launch_bounds__(256, 2) void mla_decode_mfma(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t t_lds[kWaves * kTileElems];  // 40 KB
  __shared__ float m_lds[kWaves][kH];
  __shared__ float l_lds[kWaves][kH];

  const int r = blockIdx.y;
  const int split = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;

  const int b = a.row_seq[r];
  int L = a.kv_len[r];
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const int ns = split_count(L, a.n_splits, a.min_chunk);
  if (split >= ns && !(ns == 0 && split == 0)) return;
  const int chunk = ns ? split_chunk(L, a.n_splits, a.min_chunk) : 0;
  const int t0 = split * chunk;
  const int t1 = min(L, t0 + chunk);

  // ---- Q^T operand (B of S^T): lane holds head n, channels chan(s,g)..+8.
  bf16x8_t qb[10];
  {
    const uint16_t* qa = static_cast<const uint16_t*>(a.q_abs) + r * a.qa_rs + n * a.qa_hs;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qb[s] = as_bf16x8(*reinterpret_cast<const uint4*>(qa + chan_of<C_DT>(s, g)));
    // q_pe with interleaved RoPE at table row q_rope_pos[r]
    const uint16_t* qp = static_cast<const uint16_t*>(a.q_pe) + r * a.qp_rs + n * a.qp_hs;
    int rp = a.q_rope_pos[r];
    rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
    const uint16_t* ct = static_cast<const uint16_t*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
    const uint16_t* st = static_cast<const uint16_t*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c0 = 32 * s + 8 * g;
      uint4 raw = *reinterpret_cast<const uint4*>(qp + c0);
      uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pi = c0 / 2 + j;
        float o1, o2;
        rope_pair<1>(bf16_to_f32(wv[j] & 0xFFFF), bf16_to_f32(wv[j] >> 16), bf16_to_f32(ct[pi]),
                     bf16_to_f32(st[pi]), o1, o2);
        wv[j] = f32_to_bf16(o1) | (static_cast<uint32_t>(f32_to_bf16(o2)) << 16);
      }
      qb[8 + s] = as_bf16x8(make_uint4(wv[0], wv[1], wv[2], wv[3]));
    }
  }

  f32x4_t oacc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  uint16_t* tw = t_lds + w * kTileElems;
  const int64_t cache_row0 = static_cast<int64_t>(b < 0 ? 0 : b) * a.cache_s;
  const uint16_t* kpe = static_cast<const uint16_t*>(a.kpe);

  // Loads of the K operand for the sub-tile at `base`: lane's token = base + n
  // (clamped in range; masked in the softmax).
  auto load_tile = [&](int base, uint4 (&kr)[10], float4& sc) {
    int tok = base + n;
    tok = tok < t1 ? tok : t1 - 1;
    const int64_t crow = cache_row0 + tok;
    if constexpr (C_DT == 2) {
      const uint8_t* cp = static_cast<const uint8_t*>(a.ckv) + crow * kR;
#pragma unroll
      for (int j = 0; j < 4; ++j) kr[j] = *reinterpret_cast<const uint4*>(cp + 64 * j + 16 * g);
      int tb = base + 4 * g;  // scale of the 4 tokens this lane scores
      const float* sp = a.ckv_scale + cache_row0;
      sc.x = sp[min(tb + 0, t1 - 1)];
      sc.y = sp[min(tb + 1, t1 - 1)];
      sc.z = sp[min(tb + 2, t1 - 1)];
      sc.w = sp[min(tb + 3, t1 - 1)];
    } else {
      const uint16_t* cp = static_cast<const uint16_t*>(a.ckv) + crow * kR;
#pragma unroll
      for (int s = 0; s < 8; ++s) kr[s] = *reinterpret_cast<const uint4*>(cp + 32 * s + 8 * g);
    }
    const uint16_t* pp = kpe + crow * kP;
    kr[8] = *reinterpret_cast<const uint4*>(pp + 8 * g);
    kr[9] = *reinterpret_cast<const uint4*>(pp + 32 + 8 * g);
  };

  uint4 kr[10];
  float4 sc = make_float4(1.f, 1.f, 1.f, 1.f);
  int base = t0 + kSub * w;
  if (base < t1) load_tile(base, kr, sc);

  for (; base < t1; base += kSub * kWaves) {
    // Convert the current tile into MFMA operands (e4m3 -> bf16 exactly).
    bf16x8_t ka[10];
    if constexpr (C_DT == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t l0, h0, l1, h1, l2, h2, l3, h3;
        e4m3x4_to_bf16x4(kr[j].x, l0, h0);
        e4m3x4_to_bf16x4(kr[j].y, l1, h1);
        e4m3x4_to_bf16x4(kr[j].z, l2, h2);
        e4m3x4_to_bf16x4(kr[j].w, l3, h3);
        ka[2 * j] = as_bf16x8(make_uint4(l0, h0, l1, h1));
        ka[2 * j + 1] = as_bf16x8(make_uint4(l2, h2, l3, h3));
      }
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) ka[s] = as_bf16x8(kr[s]);
    }
    ka[8] = as_bf16x8(kr[8]);
    ka[9] = as_bf16x8(kr[9]);
    const float4 sc_cur = sc;

    // Prefetch the next sub-tile of this wave.
    const int nbase = base + kSub * kWaves;
    if (nbase < t1) load_tile(nbase, kr, sc);

    // S^T = K . Q^T : lane gets head n, tokens base+4g+i.
    f32x4_t s_c = {0.f, 0.f, 0.f, 0.f}, s_p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) s_c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s], qb[s], s_c, 0, 0, 0);
#pragma unroll
    for (int s = 8; s < 10; ++s) s_p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[s], qb[s], s_p, 0, 0, 0);

    // Write the latent part transposed into the wave's LDS tile: tw[ch][tok].
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int c0 = chan_of<C_DT>(s, g);
      const uint4 v = __builtin_bit_cast(uint4, ka[s]);
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tw[(c0 + 2 * j) * kTStride + n] = static_cast<uint16_t>(wv[j] & 0xFFFF);
        tw[(c0 + 2 * j + 1) * kTStride + n] = static_cast<uint16_t>(wv[j] >> 16);
      }
    }

    // Online softmax (log2 domain).
    float x[4];
    const float scv[4] = {sc_cur.x, sc_cur.y, sc_cur.z, sc_cur.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sv = (C_DT == 2) ? (scv[i] * s_c[i] + s_p[i]) : (s_c[i] + s_p[i]);
      x[i] = (base + 4 * g + i < t1) ? sv * a.scale_log2 : -INFINITY;
    }
    float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mt = fmaxf(mt, shfl_xor_f32(mt, 16));
    mt = fmaxf(mt, shfl_xor_f32(mt, 32));
    const float m_new = fmaxf(m_run, mt);  // finite: token `base` is valid
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    uint32_t pw[2];
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float p0 = exp2f(x[2 * i] - m_new), p1 = exp2f(x[2 * i + 1] - m_new);
      // l sums the bf16-rounded weights that enter the MFMA, so a constant
      // latent row is reproduced exactly.
      const uint16_t b0 = f32_to_bf16(p0), b1 = f32_to_bf16(p1);
      psum += bf16_to_f32(b0) + bf16_to_f32(b1);
      if constexpr (C_DT == 2) {
        p0 = bf16_to_f32(b0) * scv[2 * i];
        p1 = bf16_to_f32(b1) * scv[2 * i + 1];
        pw[i] = f32_to_bf16(p0) | (static_cast<uint32_t>(f32_to_bf16(p1)) << 16);
      } else {
        pw[i] = b0 | (static_cast<uint32_t>(b1) << 16);
      }
    }
    l_part = l_part * alpha + psum;
    const s16x4_t pb = __builtin_bit_cast(s16x4_t, make_uint2(pw[0], pw[1]));

    __builtin_amdgcn_wave_barrier();
    // O^T += C^T . P^T over 16 channel blocks.
#pragma unroll
    for (int mb = 0; mb < 16; ++mb) {
      const uint2 cv = *reinterpret_cast<const uint2*>(tw + (16 * mb + n) * kTStride + 4 * g);
      const s16x4_t ca = __builtin_bit_cast(s16x4_t, cv);
      oacc[mb] = oacc[mb] * alpha;
      oacc[mb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ca, pb, oacc[mb], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- Merge the four waves.  l: reduce the lane partials of each head.
  float l_tot = l_part + shfl_xor_f32(l_part, 16);
  l_tot += shfl_xor_f32(l_tot, 32);
  if (g == 0) {
    m_lds[w][n] = m_run;
    l_lds[w][n] = l_tot;
  }
  __syncthreads();
  float mw[kWaves], M = -INFINITY;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    mw[k] = m_lds[k][n];
    M = fmaxf(M, mw[k]);
  }
  float Ltot = 0.f, my_a = 0.f;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    const float ak = (mw[k] == -INFINITY) ? 0.f : exp2f(mw[k] - M);
    Ltot += ak * l_lds[k][n];
    if (k == w) my_a = ak;
  }
  // Each wave adds its rescaled O into an fp32 LDS accumulator [16][kOStride]
  // (reusing the transposed tiles), one wave at a time.  A lane writes 4
  // consecutive channels (16 B); the padded row keeps 8-lane groups on
  // distinct banks.
  float* o_lds = reinterpret_cast<float*>(t_lds);
  __syncthreads();
#pragma unroll 1
  for (int k = 0; k < kWaves; ++k) {
    if (w == k) {
#pragma unroll
      for (int mb = 0; mb < 16; ++mb) {
        float4* dst = reinterpret_cast<float4*>(o_lds + n * kOStride + 16 * mb + 4 * g);
        float4 v = make_float4(oacc[mb][0] * my_a, oacc[mb][1] * my_a, oacc[mb][2] * my_a,
                               oacc[mb][3] * my_a);
        if (k != 0) {
          const float4 o = *dst;
          v.x += o.x;
          v.y += o.y;
          v.z += o.z;
          v.w += o.w;
        }
        *dst = v;
      }
    }
    __syncthreads();
  }

  // Thread t writes head h = t/16, channels (t%16)*16 .. +16.
  const int h = threadIdx.x >> 4, c0 = (threadIdx.x & 15) * 16;
  const float Lh = __shfl(Ltot, h, 64);  // lanes 0..15 of every wave hold head = lane
  float Mh = __shfl(M, h, 64);
  const float inv = Lh > 0.f ? 1.f / Lh : 0.f;
  const float* orow = o_lds + h * kOStride + c0;
  if (ns <= 1) {
    uint16_t* op = static_cast<uint16_t*>(a.o_lat) + r * a.o_rs + h * a.o_hs + c0;
    uint32_t pk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v0 = orow[2 * j] * inv, v1 = orow[2 * j + 1] * inv;
      pk[j] = f32_to_bf16(v0) | (static_cast<uint32_t>(f32_to_bf16(v1)) << 16);
    }
    reinterpret_cast<uint4*>(op)[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    reinterpret_cast<uint4*>(op)[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
  } else {
    const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + h;
    float* op = a.o_part + pidx * kR + c0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 v = make_float4(orow[4 * j] * inv, orow[4 * j + 1] * inv, orow[4 * j + 2] * inv,
                                   orow[4 * j + 3] * inv);
      reinterpret_cast<float4*>(op)[j] = v;
    }
    if ((threadIdx.x & 15) == 0)
      a.lse_part[pidx] = (Lh > 0.f) ? (Mh + __log2f(Lh)) * kLn2 : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Kernel 2 (fp32 models): the same maths on the VALU in fp32.  One block of
// 256 threads per (row, split); 32-token tiles staged in LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mla_decode_f32(DecodeArgs a) {
  constexpr int TT = 16;
  __shared__ float q_s[kH][kKC + 1];
  __shared__ float k_s[TT][kKC + 1];
  __shared__ float p_s[kH][TT];
  __shared__ float alpha_s[kH];
  __shared__ float m_s[kH], l_s[kH];

  const int r = blockIdx.y, split = blockIdx.x, t = threadIdx.x;
  const int b = a.row_seq[r];
  int L = a.kv_len[r];
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const int ns = split_count(L, a.n_splits, a.min_chunk);
  if (split >= ns && !(ns == 0 && split == 0)) return;
  const int chunk = ns ? split_chunk(L, a.n_splits, a.min_chunk) : 0;
  const int t0 = split * chunk, t1 = min(L, t0 + chunk);
  const int64_t row0 = static_cast<int64_t>(b < 0 ? 0 : b) * a.cache_s;

  int rp = a.q_rope_pos[r];
  rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
  const float* qa = static_cast<const float*>(a.q_abs) + r * a.qa_rs;
  const float* qp = static_cast<const float*>(a.q_pe) + r * a.qp_rs;
  const float* ct = static_cast<const float*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
  const float* st = static_cast<const float*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
  for (int i = t; i < kH * kR; i += 256) q_s[i / kR][i % kR] = qa[(i / kR) * a.qa_hs + (i % kR)];
  for (int i = t; i < kH * kP / 2; i += 256) {
    const int h = i / (kP / 2), pi = i % (kP / 2);
    float o1, o2;
    rope_pair<0>(qp[h * a.qp_hs + 2 * pi], qp[h * a.qp_hs + 2 * pi + 1], ct[pi], st[pi], o1, o2);
    q_s[h][kR + 2 * pi] = o1;
    q_s[h][kR + 2 * pi + 1] = o2;
  }
  if (t < kH) {
    m_s[t] = -INFINITY;
    l_s[t] = 0.f;
  }
  const int h_pv = t >> 4, c_pv = (t & 15) * 16;
  float o[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) o[j] = 0.f;

  const float* ckv = static_cast<const float*>(a.ckv);
  const float* kpe = static_cast<const float*>(a.kpe);
  for (int base = t0; base < t1; base += TT) {
    __syncthreads();
    for (int i = t; i < TT * kKC; i += 256) {
      const int j = i / kKC, c = i % kKC;
      const int tok = base + j;
      float v = 0.f;
      if (tok < t1) v = c < kR ? ckv[(row0 + tok) * kR + c] : kpe[(row0 + tok) * kP + (c - kR)];
      k_s[j][c] = v;
    }
    __syncthreads();
    // scores: thread -> head t/16, token t%16
    {
      const int h = t >> 4, j = t & 15;
      float acc = 0.f;
      for (int c = 0; c < kKC; ++c) acc += q_s[h][c] * k_s[j][c];
      p_s[h][j] = (base + j < t1) ? acc * a.scale_log2 : -INFINITY;
    }
    __syncthreads();
    if (t < kH) {
      float mt = -INFINITY;
      for (int j = 0; j < TT; ++j) mt = fmaxf(mt, p_s[t][j]);
      const float m_new = fmaxf(m_s[t], mt);
      const float al = exp2f(m_s[t] - m_new);
      float sum = 0.f;
      for (int j = 0; j < TT; ++j) {
        const float p = exp2f(p_s[t][j] - m_new);
        p_s[t][j] = p;
        sum += p;
      }
      l_s[t] = l_s[t] * al + sum;
      m_s[t] = m_new;
      alpha_s[t] = al;
    }
    __syncthreads();
    const float al = alpha_s[h_pv];
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) o[jj] *= al;
    for (int j = 0; j < TT; ++j) {
      const float p = p_s[h_pv][j];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) o[jj] += p * k_s[j][c_pv + jj];
    }
  }
  __syncthreads();
  const float Lh = l_s[h_pv];
  const float inv = Lh > 0.f ? 1.f / Lh : 0.f;
  if (ns <= 1) {
    float* op = static_cast<float*>(a.o_lat) + r * a.o_rs + h_pv * a.o_hs + c_pv;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) op[jj] = o[jj] * inv;
  } else {
    const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + h_pv;
    float* op = a.o_part + pidx * kR + c_pv;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) op[jj] = o[jj] * inv;
    if ((t & 15) == 0) a.lse_part[pidx] = (Lh > 0.f) ? (m_s[h_pv] + __log2f(Lh)) * kLn2 : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Kernel 3: split-KV merge.  One wavefront per (row, head), 4 per block.
// Lanes span the splits for the max / sum, then own 4 channels each.
// ---------------------------------------------------------------------------

template <int DT>
__global__ __launch_bounds__(256) void mla_merge_kernel(MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int r = blockIdx.y;
  if (h >= kH) return;
  const int ns = split_count(a.kv_len[r], a.n_splits, a.min_chunk);
  if (ns <= 1) return;  // written by the decode kernel
  const int64_t base = (static_cast<int64_t>(r) * a.n_splits) * kH + h;
  float M = -INFINITY;
  for (int s = lane; s < ns; s += 64) M = fmaxf(M, a.lse_part[base + static_cast<int64_t>(s) * kH]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) M = fmaxf(M, shfl_xor_f32(M, m));
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float wsum = 0.f;
  for (int s = 0; s < ns; ++s) {
    const int64_t pi = base + static_cast<int64_t>(s) * kH;
    const float ls = a.lse_part[pi];
    const float wgt = (ls == -INFINITY) ? 0.f : __expf(ls - M);
    wsum += wgt;
    const float4 v = reinterpret_cast<const float4*>(a.o_part + pi * kR)[lane];
    acc.x += wgt * v.x;
    acc.y += wgt * v.y;
    acc.z += wgt * v.z;
    acc.w += wgt * v.w;
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  if constexpr (DT == 0) {
    float* op = static_cast<float*>(a.o_lat) + r * a.o_rs + h * a.o_hs;
    reinterpret_cast<float4*>(op)[lane] = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  } else {
    uint16_t* op = static_cast<uint16_t*>(a.o_lat) + r * a.o_rs + h * a.o_hs;
    uint2 pk;
    pk.x = f32_to_bf16(acc.x * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.y * inv)) << 16);
    pk.y = f32_to_bf16(acc.z * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.w * inv)) << 16);
    reinterpret_cast<uint2*>(op)[lane] = pk;
  }
  if (a.lse_out && lane == 0) a.lse_out[static_cast<int64_t>(r) * kH + h] = M + __logf(wsum);
}

}  // namespace swamla

// ===========================================================================
// Host side: launchers behind the C-ABI (argument validation lives in
// mla_abi.cpp; these assume validated arguments).
// ===========================================================================
namespace swamla {

int launch_append(const AppendArgs& a, int in_dt, int c_dt, hipStream_t s) {
  const dim3 grid((a.n_tok + 3) / 4), block(256);
  if (a.n_tok == 0) return 0;
  if (in_dt == 1 && c_dt == 1) hipLaunchKernelGGL((mla_append_kernel<1, 1>), grid, block, 0, s, a);
  else if (in_dt == 1 && c_dt == 2) hipLaunchKernelGGL((mla_append_kernel<1, 2>), grid, block, 0, s, a);
  else if (in_dt == 0 && c_dt == 0) hipLaunchKernelGGL((mla_append_kernel<0, 0>), grid, block, 0, s, a);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_decode(const DecodeArgs& a, int dt, int c_dt, hipStream_t s) {
  if (a.n_rows == 0) return 0;
  const dim3 grid(a.n_splits, a.n_rows), block(256);
  if (dt == 1 && c_dt == 1) hipLaunchKernelGGL((mla_decode_mfma<1>), grid, block, 0, s, a);
  else if (dt == 1 && c_dt == 2) hipLaunchKernelGGL((mla_decode_mfma<2>), grid, block, 0, s, a);
  else if (dt == 0 && c_dt == 0) hipLaunchKernelGGL(mla_decode_f32, grid, block, 0, s, a);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_merge(const MergeArgs& a, int dt, hipStream_t s) {
  if (a.n_rows == 0 || a.n_splits <= 1) return 0;
  const dim3 grid(kH / 4, a.n_rows), block(256);
  if (dt == 1) hipLaunchKernelGGL((mla_merge_kernel<1>), grid, block, 0, s, a);
  else if (dt == 0) hipLaunchKernelGGL((mla_merge_kernel<0>), grid, block, 0, s, a);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace swamla
