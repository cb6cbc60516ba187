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
  return (c + 15) & ~15;
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
// Addressing of tokens (append) and query rows (decode / merge).
// ---------------------------------------------------------------------------
struct TokAddr {
  int b, pos, rope;
};

// Append: cache row, destination position, RoPE table row of token i.
__device__ __forceinline__ TokAddr tok_addr(const Addressing& ad, int i) {
  if (ad.start_pos) {
    const int b = i / ad.T, t = i - b * ad.T;
    const int p = ad.start_pos[b] + t;
    return {b, p, ad.rope_abs ? p : t};
  }
  return {ad.seq[i], ad.pos[i], ad.rope[i]};
}

// Decode: cache row, attended length (causal: position + 1), RoPE row of row r.
__device__ __forceinline__ TokAddr row_addr(const Addressing& ad, int r) {
  if (ad.start_pos) {
    const int b = r / ad.T, t = r - b * ad.T;
    const int p = ad.start_pos[b] + t;
    return {b, p + 1, ad.rope_abs ? p : t};
  }
  return {ad.seq[r], ad.pos[r], ad.rope[r]};
}

__device__ __forceinline__ int row_len(const Addressing& ad, int r) {
  if (ad.start_pos) {
    const int b = r / ad.T;
    return ad.start_pos[b] + (r - b * ad.T) + 1;
  }
  return ad.pos[r];
}

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
  const TokAddr ta = tok_addr(a.ad, tok);
  const int b = ta.b, pos = ta.pos, rp = ta.rope;
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
// Split-KV merge of one (row, head) by one wavefront; lane owns 4 channels.
//   o = sum_s exp(lse_s - M) o_s / sum_s exp(lse_s - M),  M = max_s lse_s
// Splits are consumed 8 at a time with all their loads in flight, merged
// online across chunks (the reference moves with each chunk's maximum).
// ---------------------------------------------------------------------------
constexpr float kLn2 = 0.6931471805599453f;

template <int DT>
__device__ __forceinline__ void merge_head(const float* __restrict__ o_part, const float* __restrict__ lse_part,
                                           int r, int h, int ns, int n_splits, void* o_lat, int64_t o_rs,
                                           int64_t o_hs, float* lse_out) {
  const int lane = threadIdx.x & 63;
  const int64_t base = static_cast<int64_t>(r) * n_splits * kH + h;  // lse index of split 0
  float M = -INFINITY, wsum = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < ns; s0 += 8) {
    float ls[8];
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int s = min(s0 + j, ns - 1);  // in range; duplicates are masked below
      const int64_t pi = base + static_cast<int64_t>(s) * kH;
      ls[j] = lse_part[pi];
      v[j] = reinterpret_cast<const float4*>(o_part + pi * kR)[lane];
    }
    float mc = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j >= ns) ls[j] = -INFINITY;
      mc = fmaxf(mc, ls[j]);
    }
    const float m_new = fmaxf(M, mc);
    if (m_new == -INFINITY) continue;  // every split so far empty
    const float alpha = (M == -INFINITY) ? 0.f : __expf(M - m_new);
    wsum *= alpha;
    acc.x *= alpha;
    acc.y *= alpha;
    acc.z *= alpha;
    acc.w *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float wgt = (ls[j] == -INFINITY) ? 0.f : __expf(ls[j] - m_new);
      wsum += wgt;
      acc.x += wgt * v[j].x;
      acc.y += wgt * v[j].y;
      acc.z += wgt * v[j].z;
      acc.w += wgt * v[j].w;
    }
    M = m_new;
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  if constexpr (DT == 0) {
    float* op = static_cast<float*>(o_lat) + r * o_rs + h * o_hs;
    reinterpret_cast<float4*>(op)[lane] = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  } else {
    uint16_t* op = static_cast<uint16_t*>(o_lat) + r * o_rs + h * o_hs;
    uint2 pk;
    pk.x = f32_to_bf16(acc.x * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.y * inv)) << 16);
    pk.y = f32_to_bf16(acc.z * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.w * inv)) << 16);
    reinterpret_cast<uint2*>(op)[lane] = pk;
  }
  if (lse_out && lane == 0) lse_out[static_cast<int64_t>(r) * kH + h] = M + __logf(wsum);
}

// ---------------------------------------------------------------------------
// Kernel 2: absorbed decode attention, bf16 MFMA (cache bf16 or e4m3).
//
// Block = NW wavefronts, one block per (query row, split).  Wave w streams
// the 16-token sub-tiles base = t0 + 16*(w + NW*i), keeping DEPTH sub-tiles
// of global loads in flight.  Per sub-tile:
//   S^T[16 tok x 16 heads] = K[16 tok x 320] . Q^T[320 x 16 heads]
//       10 x mfma_f32_16x16x32_bf16; K comes straight from 16 B global loads
//       (lane = token, 8 channels), Q^T stays in registers
//   online softmax per head, lane-local (lane owns head l%16, tokens 4g..4g+3)
//   O^T[256 ch x 16 heads] += C^T[256 x 16 tok] . P^T[16 tok x 16 heads]
//       16 x mfma_f32_16x16x16_bf16; the latent rows go to a wave-private
//       LDS tile (row-major, 544 B rows) and come back transposed through
//       ds_read_b64_tr_b16: in each 16-lane group, lane i element k is element
//       i%4 of the 8 bytes addressed by lane i/4 + 4k, so lane s points at
//       C[4g + s/4][16mb + 4(s%4)].
// The NW waves' (m, l, O) are merged through LDS at the end; rows with more
// than one split write normalised partials for mla_merge.  (Merging inside
// the decode kernel — the last block of a row combining the others' partials
// — needs device-scope release fences, which write back the whole L2 of an
// XCD per block on gfx950 and serialised the kernel; it is not done.)
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kSub = 16;                 // tokens per wave sub-tile
constexpr int kCRow = 544;               // bytes per LDS row of a latent sub-tile (512 + 32 pad)
constexpr int kCTile = kSub * kCRow;     // 8704 B per wave
constexpr int kOStride = kR + 4;         // fp32 row stride of the cross-wave merge buffer

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16x2 with the hardware RNE converter.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// Max over lanes l, l^16, l^32, l^48 (the four lane groups sharing a head)
// with the gfx950 row-swap permutes: after permlane16_swap(v, v) the pair of
// results holds v[l] and v[l^16] in some order, likewise l^32 for
// permlane32_swap, so their max is order-free.
__device__ __forceinline__ float wave_max_rows(float v) {
  const uint32_t u = f2u(v);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(u2f(r16[0]), u2f(r16[1]));
  const uint32_t u2 = f2u(v);
  const auto r32 = __builtin_amdgcn_permlane32_swap(u2, u2, false, false);
  return fmaxf(u2f(r32[0]), u2f(r32[1]));
}

constexpr float kLazy = 8.0f;  // log2 headroom before the softmax reference moves

// Channel order of the K dimension for MFMA step s (0..7) and lane group g:
// the 8 channels [chan(s,g), +8).  bf16 cache: plain order.  e4m3 cache: a
// 16 B load of 16 codes feeds steps 2j and 2j+1, so channels interleave.
template <int C_DT>
__device__ __forceinline__ int chan_of(int s, int g) {
  if constexpr (C_DT == 2) return 64 * (s >> 1) + 16 * g + 8 * (s & 1);
  return 32 * s + 8 * g;
}

// Registers of one in-flight sub-tile.  bf16: 8 x 16 B latent + 2 x 16 B
// rope.  e4m3: 4 x 16 B codes + 2 x 16 B rope + the 4 scales this lane's
// scores need.
template <int C_DT>
struct KTile;
template <>
struct KTile<1> {
  uint4 c[8];
  uint4 p[2];
};
template <>
struct KTile<2> {
  uint4 c[4];
  uint4 p[2];
  float4 sc;
};

// e4m3 x 4 (one dword) -> 4 bf16 with the hardware converter (exact: every
// e4m3fn value is a bf16 value, so keeping the high halves is exact).
__device__ __forceinline__ uint2 e4m3x4_to_bf16x4_hw(uint32_t w) {
  const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  const uint32_t a = __builtin_amdgcn_perm(f2u(lo[1]), f2u(lo[0]), 0x07060302u);
  const uint32_t b = __builtin_amdgcn_perm(f2u(hi[1]), f2u(hi[0]), 0x07060302u);
  return make_uint2(a, b);
}

template <int C_DT, int NW, int DEPTH>
__global__ __launch_bounds__(NW * 64, 2) void mla_decode_mfma(DecodeArgs a) {
  constexpr int kLdsBytes = (NW * kCTile > NW * kH * kOStride * 4) ? NW * kCTile : NW * kH * kOStride * 4;
  __shared__ __attribute__((aligned(16))) uint8_t c_lds[kLdsBytes];
  __shared__ float m_lds[NW][kH];
  __shared__ float l_lds[NW][kH];

  const int r = blockIdx.y;
  const int split = blockIdx.x;
  // The wave index is read into a scalar register so loop control below is
  // uniform (scalar branches, no exec masking) and the compiler can track
  // the in-flight loads across iterations.
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;

  const TokAddr ra = row_addr(a.ad, r);
  const int b = ra.b;
  int L = ra.pos;
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const int ns = split_count(L, a.n_splits, a.min_chunk);
  if (split >= ns && !(ns == 0 && split == 0)) return;
  const int chunk = ns ? split_chunk(L, a.n_splits, a.min_chunk) : 0;
  const int t0 = split * chunk;
  const int t1 = min(L, t0 + chunk);

  // Loads below are issued unconditionally, so every address is clamped to a
  // valid cache element: an invalid or empty row reads row 0, token 0.
  const int64_t cache_row0 = static_cast<int64_t>((b < 0 || b >= a.cache_b) ? 0 : b) * a.cache_s;
  const int t_last = t1 > 0 ? t1 - 1 : 0;
  const uint16_t* kpe = static_cast<const uint16_t*>(a.kpe);

  // Global loads of the sub-tile at `base`: lane's token = base + n (clamped
  // into range; masked in the softmax).
  auto load_tile = [&](int base, KTile<C_DT>& kt) {
    int tok = base + n;
    tok = tok < t_last ? tok : t_last;
    const int64_t crow = cache_row0 + tok;
    if constexpr (C_DT == 2) {
      const uint8_t* cp = static_cast<const uint8_t*>(a.ckv) + crow * kR;
#pragma unroll
      for (int j = 0; j < 4; ++j) kt.c[j] = *reinterpret_cast<const uint4*>(cp + 64 * j + 16 * g);
      const int tb = base + 4 * g;  // scales of the 4 tokens this lane scores
      const float* sp = a.ckv_scale + cache_row0;
      kt.sc.x = sp[min(tb + 0, t_last)];
      kt.sc.y = sp[min(tb + 1, t_last)];
      kt.sc.z = sp[min(tb + 2, t_last)];
      kt.sc.w = sp[min(tb + 3, t_last)];
    } else {
      const uint16_t* cp = static_cast<const uint16_t*>(a.ckv) + crow * kR;
#pragma unroll
      for (int s = 0; s < 8; ++s) kt.c[s] = *reinterpret_cast<const uint4*>(cp + 32 * s + 8 * g);
    }
    const uint16_t* pp = kpe + crow * kP;
    kt.p[0] = *reinterpret_cast<const uint4*>(pp + 8 * g);
    kt.p[1] = *reinterpret_cast<const uint4*>(pp + 32 + 8 * g);
  };

  // ---- Q^T operand (B of S^T): lane holds head n, channels chan(s,g)..+8.
  bf16x8_t qb[10];
  {
    const uint16_t* qa = static_cast<const uint16_t*>(a.q_abs) + r * a.qa_rs + n * a.qa_hs;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qb[s] = as_bf16x8(*reinterpret_cast<const uint4*>(qa + chan_of<C_DT>(s, g)));
    // q_pe with interleaved RoPE at the row's table position
    const uint16_t* qp = static_cast<const uint16_t*>(a.q_pe) + r * a.qp_rs + n * a.qp_hs;
    int rp = ra.rope;
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

  // Start the stream.  Every tile load is issued unconditionally (addresses
  // are clamped into the row, surplus tiles are never consumed): the wave
  // then always has exactly DEPTH tiles of loads in flight and the compiler
  // can wait on the oldest tile alone.  A conditional load would force it to
  // wait for every outstanding load, since the counter drains in order.
  // Q's loads were issued first, so waiting for them leaves the tiles in flight.
  constexpr int kStep = kSub * NW;
  const int base0 = t0 + kSub * w;
  const bool has_work = t1 > t0;  // block-uniform; false only for an empty row
  KTile<C_DT> kt[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_tile(base0 + d * kStep, kt[d]);

  f32x4_t oacc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  uint8_t* cw = c_lds + w * kCTile;
  // tr16 source address of this lane: row 4g + s/4, channel 4(s%4) (+16 mb)
  const uint8_t* tr_src = cw + (4 * g + (n >> 2)) * kCRow + 8 * (n & 3);

  auto process = [&](int base, KTile<C_DT>& kt) {
    const bool full = base + kSub <= t1;  // wave-uniform
    // MFMA operands of the latent part (e4m3 -> bf16 exactly).
    uint4 cv[8];
    float4 scv = make_float4(1.f, 1.f, 1.f, 1.f);
    if constexpr (C_DT == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint2 a0 = e4m3x4_to_bf16x4_hw(kt.c[j].x), a1 = e4m3x4_to_bf16x4_hw(kt.c[j].y);
        const uint2 a2 = e4m3x4_to_bf16x4_hw(kt.c[j].z), a3 = e4m3x4_to_bf16x4_hw(kt.c[j].w);
        cv[2 * j] = make_uint4(a0.x, a0.y, a1.x, a1.y);
        cv[2 * j + 1] = make_uint4(a2.x, a2.y, a3.x, a3.y);
      }
      scv = kt.sc;
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) cv[s] = kt.c[s];
    }
    const uint4 pv0 = kt.p[0], pv1 = kt.p[1];

    // Latent rows into the wave's LDS tile (row-major, padded rows), then
    // issue all transposed reads at once so their latency hides under the
    // score MFMAs and the softmax.
#pragma unroll
    for (int s = 0; s < 8; ++s)
      *reinterpret_cast<uint4*>(cw + n * kCRow + 2 * chan_of<C_DT>(s, g)) = cv[s];
    s16x4_t ct[16];
#pragma unroll
    for (int mb = 0; mb < 16; ++mb)
      ct[mb] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4_t*)(tr_src + 32 * mb));

    // S^T = K . Q^T : lane gets head n, tokens base+4g+i.
    f32x4_t s_c = {0.f, 0.f, 0.f, 0.f}, s_p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s)
      s_c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(cv[s]), qb[s], s_c, 0, 0, 0);
    s_p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pv0), qb[8], s_p, 0, 0, 0);
    s_p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pv1), qb[9], s_p, 0, 0, 0);

    // The registers of kt are free: refill them with the sub-tile DEPTH ahead
    // (unconditionally, see above).
    load_tile(base + DEPTH * kStep, kt);

    // Online softmax in the log2 domain with a lazily moved reference: the
    // running reference m_run only moves when a head's tile maximum exceeds
    // it by more than kLazy, so weights stay <= 2^kLazy and O is rescaled
    // rarely (the normalisation by l is exact either way).
    float x[4];
    const float sc4[4] = {scv.x, scv.y, scv.z, scv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sv = (C_DT == 2) ? (sc4[i] * s_c[i] + s_p[i]) : (s_c[i] + s_p[i]);
      x[i] = sv * a.scale_log2;
    }
    if (!full) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (base + 4 * g + i >= t1) x[i] = -INFINITY;
    }
    float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mt = wave_max_rows(mt);  // max over lanes n, n+16, n+32, n+48 (one head)
    if (__any(mt > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, mt);  // finite: token `base` is valid
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
#pragma unroll
      for (int mb = 0; mb < 16; ++mb) oacc[mb] = oacc[mb] * alpha;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = exp2f(x[i] - m_run);
    // bf16 weights for the MFMA (hardware RNE); l sums exactly those values,
    // so a constant latent row is reproduced exactly.
    const uint32_t w01 = pack_bf16x2(p[0], p[1]), w23 = pack_bf16x2(p[2], p[3]);
    l_part += (u2f(w01 << 16) + u2f(w01 & 0xFFFF0000u)) + (u2f(w23 << 16) + u2f(w23 & 0xFFFF0000u));
    uint2 pw;
    if constexpr (C_DT == 2) {
      pw.x = pack_bf16x2(u2f(w01 << 16) * sc4[0], u2f(w01 & 0xFFFF0000u) * sc4[1]);
      pw.y = pack_bf16x2(u2f(w23 << 16) * sc4[2], u2f(w23 & 0xFFFF0000u) * sc4[3]);
    } else {
      pw = make_uint2(w01, w23);
    }
    const s16x4_t pb = __builtin_bit_cast(s16x4_t, pw);

    // O^T += C^T . P^T over 16 channel blocks.
#pragma unroll
    for (int mb = 0; mb < 16; ++mb)
      oacc[mb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ct[mb], pb, oacc[mb], 0, 0, 0);
  };

  // Sub-tiles of this wave: full groups of DEPTH in the loop, the remainder
  // after it; every branch is uniform.  Surplus refills at the end of the
  // stream re-read the wave's last row (cache hits) and drain in order right
  // behind the real tiles.
  const int n_sub = (has_work && base0 < t1) ? (t1 - base0 + kStep - 1) / kStep : 0;
  int it = 0;
  for (; it + DEPTH <= n_sub; it += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) process(base0 + (it + d) * kStep, kt[d]);
  }
#pragma unroll
  for (int d = 0; d < DEPTH - 1; ++d)
    if (it + d < n_sub) process(base0 + (it + d) * kStep, kt[d]);

  // ---- Merge the NW waves.  l: reduce the lane partials of each head.
  float l_tot = l_part + shfl_xor_f32(l_part, 16);
  l_tot += shfl_xor_f32(l_tot, 32);
  if (g == 0) {
    m_lds[w][n] = m_run;
    l_lds[w][n] = l_tot;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int k = 0; k < NW; ++k) M = fmaxf(M, m_lds[k][n]);
  float Ltot = 0.f, my_a = 0.f;
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    const float mk = m_lds[k][n];
    const float ak = (mk == -INFINITY) ? 0.f : exp2f(mk - M);
    Ltot += ak * l_lds[k][n];
    if (k == w) my_a = ak;
  }
  // Each wave stores its rescaled O into its own fp32 LDS region
  // [16][kOStride] (reusing the tiles); after one barrier every thread sums
  // the NW regions for its channels.  A lane stores 4 consecutive channels
  // (16 B); the padded rows keep 8-lane groups on distinct banks.
  float* o_lds = reinterpret_cast<float*>(c_lds);
  {
    float* mine = o_lds + w * (kH * kOStride);
#pragma unroll
    for (int mb = 0; mb < 16; ++mb)
      *reinterpret_cast<float4*>(mine + n * kOStride + 16 * mb + 4 * g) =
          make_float4(oacc[mb][0] * my_a, oacc[mb][1] * my_a, oacc[mb][2] * my_a, oacc[mb][3] * my_a);
  }
  __syncthreads();

  // Thread t writes head h, CPT channels.
  constexpr int TPH = NW * 64 / kH, CPT = kR / TPH;
  const int h = threadIdx.x / TPH, c0 = (threadIdx.x % TPH) * CPT;
  const float Lh = __shfl(Ltot, h, 64);  // lanes 0..15 of every wave hold head = lane
  const float Mh = __shfl(M, h, 64);
  const float inv = Lh > 0.f ? 1.f / Lh : 0.f;
  float orow[CPT];
#pragma unroll
  for (int j = 0; j < CPT / 4; ++j) {
    float4 acc = *reinterpret_cast<const float4*>(o_lds + h * kOStride + c0 + 4 * j);
#pragma unroll
    for (int k = 1; k < NW; ++k) {
      const float4 v = *reinterpret_cast<const float4*>(o_lds + k * (kH * kOStride) + h * kOStride + c0 + 4 * j);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    orow[4 * j] = acc.x;
    orow[4 * j + 1] = acc.y;
    orow[4 * j + 2] = acc.z;
    orow[4 * j + 3] = acc.w;
  }
  if (ns <= 1) {
    uint16_t* op = static_cast<uint16_t*>(a.o_lat) + r * a.o_rs + h * a.o_hs + c0;
#pragma unroll
    for (int j = 0; j < CPT / 8; ++j) {
      uint32_t pk[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        pk[k] = f32_to_bf16(orow[8 * j + 2 * k] * inv) |
                (static_cast<uint32_t>(f32_to_bf16(orow[8 * j + 2 * k + 1] * inv)) << 16);
      reinterpret_cast<uint4*>(op)[j] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
    return;
  }
  const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + h;
  float* op = a.o_part + pidx * kR + c0;
#pragma unroll
  for (int j = 0; j < CPT / 4; ++j)
    reinterpret_cast<float4*>(op)[j] = make_float4(orow[4 * j] * inv, orow[4 * j + 1] * inv,
                                                   orow[4 * j + 2] * inv, orow[4 * j + 3] * inv);
  if ((threadIdx.x % TPH) == 0) a.lse_part[pidx] = (Lh > 0.f) ? (Mh + __log2f(Lh)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Kernel 2 (fp32 models): the same maths on the VALU in fp32.  One block of
// 256 threads per (row, split); 16-token tiles staged in LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mla_decode_f32(DecodeArgs a) {
  constexpr int TT = 16;
  __shared__ float q_s[kH][kKC + 1];
  __shared__ float k_s[TT][kKC + 1];
  __shared__ float p_s[kH][TT];
  __shared__ float alpha_s[kH];
  __shared__ float m_s[kH], l_s[kH];

  const int r = blockIdx.y, split = blockIdx.x, t = threadIdx.x;
  const TokAddr ra = row_addr(a.ad, r);
  const int b = ra.b;
  int L = ra.pos;
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const int ns = split_count(L, a.n_splits, a.min_chunk);
  if (split >= ns && !(ns == 0 && split == 0)) return;
  const int chunk = ns ? split_chunk(L, a.n_splits, a.min_chunk) : 0;
  const int t0 = split * chunk, t1 = min(L, t0 + chunk);
  const int64_t row0 = static_cast<int64_t>(b < 0 ? 0 : b) * a.cache_s;

  int rp = ra.rope;
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
    {  // scores: thread -> head t/16, token t%16
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
    return;
  }
  const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + h_pv;
  float* op = a.o_part + pidx * kR + c_pv;
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) op[jj] = o[jj] * inv;
  if ((t & 15) == 0) a.lse_part[pidx] = (Lh > 0.f) ? (m_s[h_pv] + __log2f(Lh)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Kernel 3: split-KV merge, one wavefront per (row, head).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(64) void mla_merge_kernel(MergeArgs a) {
  const int h = blockIdx.x, r = blockIdx.y;
  const int ns = split_count(row_len(a.ad, r), a.n_splits, a.min_chunk);
  if (ns <= 1) return;  // written by the decode kernel
  merge_head<DT>(a.o_part, a.lse_part, r, h, ns, a.n_splits, a.o_lat, a.o_rs, a.o_hs, a.lse_out);
}

}  // namespace swamla

// ===========================================================================
// Launchers behind the C-ABI (argument validation lives in mla_abi.cpp; these
// assume validated arguments).
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
  const dim3 grid(a.n_splits, a.n_rows);
  if (dt == 1 && c_dt == 1) hipLaunchKernelGGL((mla_decode_mfma<1, 4, 2>), grid, dim3(256), 0, s, a);
  else if (dt == 1 && c_dt == 2) hipLaunchKernelGGL((mla_decode_mfma<2, 4, 2>), grid, dim3(256), 0, s, a);
  else if (dt == 0 && c_dt == 0) hipLaunchKernelGGL(mla_decode_f32, grid, dim3(256), 0, s, a);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_merge(const MergeArgs& a, int dt, hipStream_t s) {
  if (a.n_rows == 0 || a.n_splits <= 1) return 0;
  const dim3 grid(kH, a.n_rows), block(64);
  if (dt == 1) hipLaunchKernelGGL((mla_merge_kernel<1>), grid, block, 0, s, a);
  else if (dt == 0) hipLaunchKernelGGL((mla_merge_kernel<0>), grid, block, 0, s, a);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace swamla
