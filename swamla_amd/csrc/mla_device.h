// mla_device.h — device code shared by the gfx950 kernels: geometry and tile
// constants, the per-op-rounded arithmetic of the append path (LayerNorm,
// RoPE, e4m3 encoding), bf16 / e4m3 conversions, MFMA operand helpers, the
// LDS-only barrier and the non-temporal 16-byte load.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "numerics.h"

namespace swamla {

constexpr int kP = 64;
constexpr int kH = 16;
// Latent rows: kv_lora_rank R is stored padded to R_pad = 64 NB channels
// (NB = ceil(R / 64), at most kMaxNB); channels R .. R_pad - 1 hold zeros.
// Kernels are instantiated per NB; R itself only enters the LayerNorm and
// the masking of query padding.

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

// The arithmetic below is shared by the append kernel and the decode kernel's
// fused one-token append, so both write identical bits.

// LayerNorm of one latent row held by a wavefront, lane owning the K = R_pad /
// 64 channels K*lane .. K*lane + K - 1.  Channels >= R are padding: they take
// no part in the statistics and come out as exactly 0.  Every multiply / add
// is rounded on its own: the result must reproduce the fixed-order fp64
// statement exactly.  Statistics in fp64; fixed order: in-lane left to
// right, then xor butterfly 1,2,4,...,32 (every lane ends with the same total),
// times inv_r = fl64(1 / R) (exactly 2^-8 for R = 256).
template <int K>
__device__ __forceinline__ void layernorm_lane(const double (&x)[K], const double (&wt)[K], const double (&bs)[K],
                                               int R, double inv_r, int lane, float eps, double (&y)[K]) {
#pragma clang fp contract(off)
  bool v[K];
#pragma unroll
  for (int i = 0; i < K; ++i) v[i] = K * lane + i < R;
  double s = v[0] ? x[0] : 0.0;
#pragma unroll
  for (int i = 1; i < K; ++i) s = s + (v[i] ? x[i] : 0.0);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) s = s + shfl_xor_f64(s, m);
  const double mean = s * inv_r;
  double d[K];
#pragma unroll
  for (int i = 0; i < K; ++i) d[i] = v[i] ? x[i] - mean : 0.0;
  double q = d[0] * d[0];
#pragma unroll
  for (int i = 1; i < K; ++i) q = q + d[i] * d[i];
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) q = q + shfl_xor_f64(q, m);
  const double var = q * inv_r;
  // correctly rounded square root and IEEE division
  const double rstd = 1.0 / __dsqrt_rn(var + static_cast<double>(eps));
#pragma unroll
  for (int i = 0; i < K; ++i) y[i] = v[i] ? (d[i] * rstd) * wt[i] + bs[i] : 0.0;
}

// bf16 cache: each channel rounded once from fp64.
template <int K>
__device__ __forceinline__ void encode_bf16_lane(const double (&y)[K], uint16_t (&o)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) o[i] = f64_to_bf16(y[i]);
}

// e4m3 per token: y is first rounded to bf16 (the value a bf16 cache would
// hold), amax over the token, scale = max(amax,1e-12)/448, code = RNE(y/scale).
// Padding channels (y = 0) encode as 0.
template <int K>
__device__ __forceinline__ void encode_e4m3_lane(const double (&y)[K], uint8_t (&codes)[K], float& scale) {
  float yb[K];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    yb[i] = bf16_to_f32(f64_to_bf16(y[i]));
    amax = fmaxf(amax, fabsf(yb[i]));
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) amax = fmaxf(amax, shfl_xor_f32(amax, m));
  scale = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
#pragma unroll
  for (int i = 0; i < K; ++i) codes[i] = f32_to_e4m3(__fdiv_rn(yb[i], scale));
}

// K consecutive 16-bit / 8-bit values of one lane, moved with the widest
// vector the lane's offset (a multiple of K elements) keeps aligned.
template <int K, typename U>
__device__ __forceinline__ void load_lane(const U* p, U (&v)[K]) {
  constexpr int B = K * static_cast<int>(sizeof(U));
  if constexpr (B % 16 == 0) {
#pragma unroll
    for (int c = 0; c < B / 16; ++c) {
      const uint4 t = reinterpret_cast<const uint4*>(p)[c];
      __builtin_memcpy(reinterpret_cast<uint8_t*>(v) + 16 * c, &t, 16);
    }
  } else if constexpr (B % 8 == 0) {
#pragma unroll
    for (int c = 0; c < B / 8; ++c) {
      const uint2 t = reinterpret_cast<const uint2*>(p)[c];
      __builtin_memcpy(reinterpret_cast<uint8_t*>(v) + 8 * c, &t, 8);
    }
  } else if constexpr (B % 4 == 0) {
#pragma unroll
    for (int c = 0; c < B / 4; ++c) {
      const uint32_t t = reinterpret_cast<const uint32_t*>(p)[c];
      __builtin_memcpy(reinterpret_cast<uint8_t*>(v) + 4 * c, &t, 4);
    }
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) v[i] = p[i];
  }
}
template <int K, typename U>
__device__ __forceinline__ void store_lane(U* p, const U (&v)[K]) {
  constexpr int B = K * static_cast<int>(sizeof(U));
  if constexpr (B % 16 == 0) {
#pragma unroll
    for (int c = 0; c < B / 16; ++c) {
      uint4 t;
      __builtin_memcpy(&t, reinterpret_cast<const uint8_t*>(v) + 16 * c, 16);
      reinterpret_cast<uint4*>(p)[c] = t;
    }
  } else if constexpr (B % 8 == 0) {
#pragma unroll
    for (int c = 0; c < B / 8; ++c) {
      uint2 t;
      __builtin_memcpy(&t, reinterpret_cast<const uint8_t*>(v) + 8 * c, 8);
      reinterpret_cast<uint2*>(p)[c] = t;
    }
  } else if constexpr (B % 4 == 0) {
#pragma unroll
    for (int c = 0; c < B / 4; ++c) {
      uint32_t t;
      __builtin_memcpy(&t, reinterpret_cast<const uint8_t*>(v) + 4 * c, 4);
      reinterpret_cast<uint32_t*>(p)[c] = t;
    }
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) p[i] = v[i];
  }
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kSub = 16;                   // tokens per wave in a tile
constexpr int kWaves = 4;                  // waves per block
constexpr int kTileTok = kSub * kWaves;    // 64 tokens per lockstep tile
constexpr int kPeRow = 2 * kP + 16;        // 144 B per LDS rope row
constexpr int kPeBytes = kTileTok * kPeRow;  // 9216 B

// Latent geometry of an instance: R_pad = 64 NB channels, LDS latent rows of
// 2 R_pad + PAD bytes.  The decode kernel uses PAD = 16 (528 B for NB = 4:
// the 16 rows of a 16-byte-per-lane operand read fall on distinct 16-byte
// bank slots).  The prefill kernel, where every wave also reads the whole
// tile transposed (32 bytes of each of 16 rows per instruction), uses
// PAD = 32: measured 6-8 % faster there (B = 4 and 32 x 4096 tokens), and
// no faster for decode.
template <int NB, int PAD = 16>
struct LatGeo {
  static constexpr int RP = 64 * NB;
  static constexpr int CRow = 2 * RP + PAD;
  static constexpr int CBytes = kTileTok * CRow;
};
constexpr int kPRow = 2 * kTileTok + 8;    // bytes per head row of P (128 + 8 pad: the 16 heads
                                           // of an 8-byte access fall on distinct banks)

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }
__device__ __forceinline__ bf16x8_t cat_bf16x8(s16x4_t lo, s16x4_t hi) {
  const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
  return as_bf16x8(make_uint4(a.x, a.y, b.x, b.y));
}

// The first n (clamped to 0..8) of eight packed bf16 kept, the rest zeroed.
__device__ __forceinline__ uint4 mask_bf16x8(uint4 v, int n) {
  auto m = [n](int k) {
    return (2 * k < n ? 0x0000FFFFu : 0u) | (2 * k + 1 < n ? 0xFFFF0000u : 0u);
  };
  return make_uint4(v.x & m(0), v.y & m(1), v.z & m(2), v.w & m(3));
}

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

// Workgroup barrier that orders LDS only: global loads stay in flight across
// it (a full fence would also wait for them).  The release half completes
// this wave's earlier LDS reads and writes before the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Registers of one in-flight tile (this wave's 16 tokens), loaded as whole
// lines: element s of c covers tokens 8(s&1)..+8, bytes 128(s>>1)..+128 of
// the latent rows (lane: token l%8, 16 B at 16(l/8)); p[j] the same for
// rope rows, tokens 8j..+8.  bf16 rows of R_pad = 64 NB channels are NB
// segments; e4m3 rows are ceil(NB / 2) segments of codes (for odd NB the last
// one is half a row: its upper lanes re-read the row's first bytes, unused),
// plus the 4 scales this lane's scores need.
template <int C_DT, int NB>
struct KTile;
template <int NB>
struct KTile<1, NB> {
  uint4 c[2 * NB];
  uint4 p[2];
};
template <int NB>
struct KTile<2, NB> {
  uint4 c[2 * ((NB + 1) / 2)];
  uint4 p[2];
  float4 sc;
};

// e4m3 x 4 (one dword) -> 4 bf16 with gfx950's packed converter, two codes
// per instruction (scale 1: exact, since every e4m3fn value is a bf16 value).
// Bit-identical, NaN codes included, to converting each pair to f32 and
// keeping the high halves, over all 65,536 code pairs.
__device__ __forceinline__ uint2 e4m3x4_to_bf16x4_hw(uint32_t w) {
  const uint32_t a = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  const uint32_t b = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  return make_uint2(a, b);
}

// One e4m3 code as bf16 bits (exact: every e4m3fn value is a bf16 value).
__device__ __forceinline__ uint16_t e4m3_to_bf16_bits(uint8_t c) {
  return static_cast<uint16_t>(f2u(e4m3_to_f32(c)) >> 16);
}

// 16-byte global load marked non-temporal: the cache is streamed once, and
// the non-temporal hint keeps it from thrashing the vector L1 (measured
// ~10 % more read bandwidth for this kernel on MI355X).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}

}  // namespace swamla
