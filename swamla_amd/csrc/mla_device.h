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

__device__ __forceinline__ float shfl_xor_f32(float v, int m) { return __shfl_xor(v, m, 64); }

// The arithmetic below is shared by the append kernel and the decode kernel's
// fused one-token append, so both write identical bits.

// ---------------------------------------------------------------------------
// kv_norm exactly as PyTorch's CPU LayerNorm computes it (the reference's
// `self.kv_norm(kv)`, models/mla.py:107, :409).  The statistics are a
// vectorised fp32 Welford pass, every product and sum rounded where ATen's
// compiled CPU kernel rounds it (restated and pinned bit for bit against
// torch on the host by the oracle's aten_layernorm.c):
//   * input vectors of V values (16 for bf16 input, 8 for fp32) are HV = V/8
//     float vectors of 8 lanes; n = R / V whole vectors in chunks of 16;
//   * one Welford stream per (chunk, half, lane k) over the chunk's vectors j:
//       d = x - m1;  m1 = fma(d, fl(1/(j+1)), m1);  m2 = fma(d, x - m1, m2)
//   * the streams merge, chunk by chunk and half by half, into a binary-counter
//     stack of 8-lane accumulators (depth ceil(log2(chunks)), at least 1):
//       c = fl(cnt_add / cnt);  dc = d * c;  m1 += dc;
//       m2 = fma(dc, d * fl(cnt_old), m2 + m2_add)
//   * the R - nV tail values run a scalar Welford (m1 += d / cnt), and the 8
//     lanes, n HV values each, merge into it one by one:
//       m1 = fma(d, c, m1);  m2 = m2 + fma((d * d) * c, fl(cnt_old), m2_add)
//   * var = m2 / R;  rstd = 1 / sqrt(var + eps).
// One wavefront per row: lanes 0..31 run the streams (chunk / half / lane from
// the lane index), the stack merges run in every lane for its k = lane % 8,
// the tail and the lane merges run uniformly in all lanes.  Kernel ranks are
// R <= 512: at most 2 chunks for bf16 (depth 1) and 4 for fp32 (depth 2).
struct LnStats {
  float mean, rstd;
};

// Correctly rounded fp32 square root.  On gfx950 the compiler lowers both
// sqrtf and __fsqrt_rn to v_sqrt_f32, whose result is not always the nearest
// float.  The estimate s is within an ulp or two of the root; the root lies
// below s's lower midpoint iff x is below that midpoint's square (likewise
// above), and a midpoint of two floats (25 significant bits) squares exactly
// in fp64.  A float's root is never exactly a midpoint, so there are no ties.
__device__ __forceinline__ float sqrt_rn_f32(float x) {
#pragma clang fp contract(off)
  float s = __builtin_sqrtf(x);
  if (!(x > 0.f) || !(x < INFINITY)) return s;  // 0, negative, NaN, inf: as the hardware gives
  const double xd = static_cast<double>(x);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const float dn = u2f(f2u(s) - 1u), up = u2f(f2u(s) + 1u);
    const double mlo = 0.5 * (static_cast<double>(dn) + static_cast<double>(s));
    const double mhi = 0.5 * (static_cast<double>(s) + static_cast<double>(up));
    s = xd < mlo * mlo ? dn : (xd > mhi * mhi ? up : s);
  }
  return s;
}

__device__ __forceinline__ void ln_stack_merge(int add_cnt, float a1, float a2, int& cnt, float& m1, float& m2) {
#pragma clang fp contract(off)
  const int tot = cnt + add_cnt;
  const float c = tot == 0 ? 0.f : __fdiv_rn(static_cast<float>(add_cnt), static_cast<float>(tot));
  const float d = a1 - m1;
  const float dc = d * c;
  const float base = m2 + a2;
  m2 = __builtin_fmaf(dc, d * static_cast<float>(cnt), base);
  m1 = m1 + dc;
  cnt = tot;
}

// The row's values as the statistics read them: lane l < 32 holds its
// stream's (up to 16) values, lane i < R - nV the i-th tail value, as raw bits
// (bf16 in the low half, or fp32).
struct LnRow {
  uint32_t xs[16];
  uint32_t xt;
};

template <int IN_DT>
__device__ __forceinline__ float ln_val(uint32_t raw) {
  if constexpr (IN_DT == 1) return u2f(raw << 16);
  else return u2f(raw);
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Vector-memory loads as inline assembly, for kernels that keep count of their
// loads in flight themselves: the compiler's wait insertion does not see these,
// so it neither waits for them nor (missing the global_load_lds tile copies
// issued after them) drains every copy in flight before their first use.  The
// caller waits with an explicit s_waitcnt vmcnt and then passes the results
// through vm_release(), which keeps every use below that wait.
typedef uint32_t vm_u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t vm_u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t vm_u32x4_t __attribute__((ext_vector_type(4)));
template <int W>
__device__ __forceinline__ void vm_load(const void* p, uint32_t (&v)[W]) {
  static_assert(W >= 1 && W <= 4, "1 to 4 words");
  if constexpr (W == 1) {
    asm volatile("global_load_dword %0, %1, off" : "=v"(v[0]) : "v"(p));
  } else if constexpr (W == 2) {
    vm_u32x2_t t;
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(t) : "v"(p));
    v[0] = t[0], v[1] = t[1];
  } else if constexpr (W == 3) {
    vm_u32x3_t t;
    asm volatile("global_load_dwordx3 %0, %1, off" : "=v"(t) : "v"(p));
    v[0] = t[0], v[1] = t[1], v[2] = t[2];
  } else {
    vm_u32x4_t t;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(t) : "v"(p));
    v[0] = t[0], v[1] = t[1], v[2] = t[2], v[3] = t[3];
  }
}
__device__ __forceinline__ uint32_t vm_load_u16(const void* p) {
  uint32_t v;
  asm volatile("global_load_ushort %0, %1, off" : "=v"(v) : "v"(p));
  return v;
}
template <int W>
__device__ __forceinline__ void vm_release(uint32_t (&v)[W]) {
#pragma unroll
  for (int i = 0; i < W; ++i) asm volatile("" : "+v"(v[i]));
}

// LDS bytes ln_gather needs: the row (64 K elements) and the spans its
// reads touch (16 vectors past each lane's stream start, values unused).
template <int IN_DT>
constexpr int ln_stage_bytes() {
  return IN_DT == 1 ? 2048 : 4096;
}

namespace ln_detail {
// The LDS traffic is inline assembly so that the compiler, which cannot tell
// this area from a ring buffer still being filled by global_load_lds in the
// decode kernel, does not drain every load in flight before it.
template <int ES, int OFF>
__device__ __forceinline__ void write(uint32_t addr, uint32_t v) {
  if constexpr (ES == 2) asm volatile("ds_write_b16 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(OFF) : "memory");
  else asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(OFF) : "memory");
}
template <int ES, int OFF>
__device__ __forceinline__ uint32_t read(uint32_t addr) {
  uint32_t v;
  if constexpr (ES == 2) asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  else asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <int ES, int K, int W, int M>
__device__ __forceinline__ void write_lane(uint32_t addr, const uint32_t (&xw)[W]) {
  if constexpr (M < K) {
    if constexpr (ES == 4) write<4, 4 * M>(addr, xw[M]);
    else if constexpr (K % 2 == 0 && M % 2 == 0) write<4, 2 * M>(addr, xw[M / 2]);  // a pair per word
    else if constexpr (K % 2 != 0) write<2, 2 * M>(addr, (M & 1) ? (xw[M / 2] >> 16) : xw[M / 2]);
    write_lane<ES, K, W, M + 1>(addr, xw);
  }
}
template <int ES, int STEP, int J>
__device__ __forceinline__ void read_stream(uint32_t addr, uint32_t (&xs)[16]) {
  if constexpr (J < 16) {
    xs[J] = read<ES, J * STEP>(addr);
    read_stream<ES, STEP, J + 1>(addr, xs);
  }
}
}  // namespace ln_detail

// Builds the statistics' layout from the row as the wavefront already holds
// it — lane l owning channels K l .. K l + K - 1 as raw words (K bf16 values
// packed two per word, or K fp32 words) — by staging the row in `buf`
// (ln_stage_bytes<IN_DT>() bytes of LDS that only this wavefront touches
// while this runs), so the LayerNorm reads the row from memory once.  A
// wavefront's LDS operations complete in order, so the reads see the writes.
//
// G = 16: the row is held by an aligned group of 16 lanes (bf16, R <= 256,
// K = 16; lane = the lane in the group), and `buf` needs ln_stage_g16_bytes:
// the 512-byte row and the tail reads past it.
constexpr int ln_stage_g16_bytes() { return 544; }
template <int IN_DT, int K, int G = 64>
__device__ __forceinline__ LnRow ln_gather(const uint32_t (&xw)[IN_DT == 1 ? (K + 1) / 2 : K], int R, int lane,
                                           lds_u8* buf) {
  constexpr int V = IN_DT == 1 ? 16 : 8;
  constexpr int HV = V / 8;
  constexpr int ES = IN_DT == 1 ? 2 : 4;  // bytes per element
  constexpr int W = IN_DT == 1 ? (K + 1) / 2 : K;
  static_assert(G == 64 ? 64 * K * ES <= ln_stage_bytes<IN_DT>() : (G == 16 && IN_DT == 1 && K == 16),
                "staging area");
  const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(buf));
  ln_detail::write_lane<ES, K, W, 0>(base + ES * K * lane, xw);
  // the lane of stream (chunk sc, half sh, lane sk) reads elements s0 + j V,
  // j = 0..15, s0 = 16 V sc + 8 sh + sk (those past the stream's count, and
  // every read of a lane without a stream, land in the staging area and are
  // ignored); lane i reads tail value n V + i
  const int n = R / V;
  const int sc = lane / (8 * HV), sh = (lane >> 3) & (HV - 1), sk = lane & 7;
  LnRow x;
  ln_detail::read_stream<ES, ES * V, 0>(base + ES * (sc * 16 * V + 8 * sh + sk), x.xs);
  x.xt = ln_detail::read<ES, 0>(base + ES * (n * V + lane));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int j = 0; j < 16; ++j) asm volatile("" : "+v"(x.xs[j]));
  asm volatile("" : "+v"(x.xt));
  return x;
}

// The value of v on lane idx of the caller's lane group: the whole wavefront
// (G = 64; idx uniform) or the caller's aligned group of 16 lanes (G = 16).
template <int G>
__device__ __forceinline__ uint32_t grp_lane(uint32_t v, int idx, int lane) {
  static_assert(G == 64 || G == 16, "lane groups of 64 or 16");
  if constexpr (G == 64) return __builtin_amdgcn_readlane(v, idx);
  else return static_cast<uint32_t>(__shfl(static_cast<int>(v), (lane & ~(G - 1)) + idx, 64));
}

// The statistics of one row held by a group of G lanes (lane = the lane in
// the wavefront; the group's lanes play lanes 0 .. G-1 of the description
// above).  G = 16 covers rows whose streams fit the group: one chunk, i.e.
// R < 272 for bf16 input (the 4-tokens-per-wavefront append at R_pad = 256).
template <int IN_DT, int G = 64>
__device__ __forceinline__ LnStats aten_ln_stats(const LnRow& x, int R, float eps, int lane) {
#pragma clang fp contract(off)
  constexpr int V = IN_DT == 1 ? 16 : 8;         // values per input vector
  constexpr int HV = V / 8;                       // 8-lane float vectors per input vector
  constexpr int kMaxChunks = G == 16 ? 16 / (8 * HV) : (IN_DT == 1 ? 4 : 8);  // R <= 1024 (G = 64)
  const int gbase = lane & ~(G - 1);
  const int n = R / V;
  const int chunks = (n + 15) >> 4;
  // --- streams (lanes 0..31 of the group; a lane past the chunks has none)
  const int sc = (lane & (G - 1)) / (8 * HV);
  int scnt = n - 16 * sc;
  scnt = scnt < 0 ? 0 : (scnt > 16 ? 16 : scnt);
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    if (j < scnt) {
      const float xv = ln_val<IN_DT>(x.xs[j]);
      const float c = __fdiv_rn(1.0f, static_cast<float>(j + 1));
      const float d = xv - s1;
      s1 = __builtin_fmaf(d, c, s1);
      s2 = __builtin_fmaf(d, xv - s1, s2);
    }
  }
  // --- stack merges (lane k = lane % 8 keeps lane k's accumulators): a
  // binary counter over the chunks, depth ceil(log2(chunks)) (at least 1)
  const int k = lane & 7;
  constexpr int kMaxDepth = kMaxChunks <= 2 ? 1 : (kMaxChunks <= 4 ? 2 : 3);
  const int depth = chunks <= 2 ? 1 : (chunks <= 4 ? 2 : 3);
  int sc_[kMaxDepth];
  float s1_[kMaxDepth], s2_[kMaxDepth];
#pragma unroll
  for (int j = 0; j < kMaxDepth; ++j) {
    sc_[j] = 0;
    s1_[j] = 0.f;
    s2_[j] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    if (i < chunks) {  // uniform
      const int ci = (n - 16 * i) < 16 ? n - 16 * i : 16;
#pragma unroll
      for (int h = 0; h < HV; ++h) {
        const int src = (i * HV + h) * 8 + k;
        ln_stack_merge(ci, __shfl(s1, gbase + src, 64), __shfl(s2, gbase + src, 64), sc_[0], s1_[0], s2_[0]);
      }
      // carry: level j - 1 moves into level j while the counter's low bits are zero
      int carry = i + 1;
      bool go = true;
#pragma unroll
      for (int j = 1; j < kMaxDepth; ++j) {
        go = go && j < depth && (carry & 1) == 0;
        if (go) {
          ln_stack_merge(sc_[j - 1], s1_[j - 1], s2_[j - 1], sc_[j], s1_[j], s2_[j]);
          sc_[j - 1] = 0;
          s1_[j - 1] = 0.f;
          s2_[j - 1] = 0.f;
        }
        carry >>= 1;
      }
    }
  }
#pragma unroll
  for (int j = 1; j < kMaxDepth; ++j)
    if (j < depth) ln_stack_merge(sc_[j], s1_[j], s2_[j], sc_[0], s1_[0], s2_[0]);
  const float a1 = s1_[0], a2 = s2_[0];
  // --- scalar tail, then the 8 lanes (values uniform across the wave)
  int cnt = 0;
  float m1 = 0.f, m2 = 0.f;
  for (int i = 0; i < R - n * V; ++i) {  // uniform, < V
    const float xv = ln_val<IN_DT>(grp_lane<G>(x.xt, i, lane));
    const float d = xv - m1;
    ++cnt;
    m1 = m1 + __fdiv_rn(d, static_cast<float>(cnt));
    m2 = __builtin_fmaf(d, xv - m1, m2);
  }
  const int per_lane = n * HV;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const float l1 = u2f(grp_lane<G>(f2u(a1), kk, lane));
    const float l2 = u2f(grp_lane<G>(f2u(a2), kk, lane));
    const int tot = cnt + per_lane;
    const float c = tot == 0 ? 0.f : __fdiv_rn(static_cast<float>(per_lane), static_cast<float>(tot));
    const float d = l1 - m1;
    m1 = __builtin_fmaf(d, c, m1);
    const float t = (d * d) * c;
    m2 = m2 + __builtin_fmaf(t, static_cast<float>(cnt), l2);
    cnt = tot;
  }
  const float var = __fdiv_rn(m2, static_cast<float>(R));
  return LnStats{m1, __fdiv_rn(1.0f, sqrt_rn_f32(var + eps))};
}

// The affine part per channel (fp32 result, before rounding to the cache
// dtype): bf16 input y = fma(fma(x, rstd, -rstd * mean), w, b); fp32 input
// y = fma((x - mean) * rstd, w, b).
template <int IN_DT>
__device__ __forceinline__ float aten_ln_affine(float x, float w, float b, const LnStats& st) {
#pragma clang fp contract(off)
  if constexpr (IN_DT == 1) {
    const float bias = -st.rstd * st.mean;
    return __builtin_fmaf(__builtin_fmaf(x, st.rstd, bias), w, b);
  } else {
    return __builtin_fmaf((x - st.mean) * st.rstd, w, b);
  }
}

// LayerNorm of one latent row held by a wavefront, lane owning the K = R_pad /
// 64 channels K*lane .. K*lane + K - 1 (x, w, b as loaded, in fp32).  Channels
// >= R are padding and come out as exactly 0.
template <int IN_DT, int K>
__device__ __forceinline__ void layernorm_lane(const float (&x)[K], const float (&wt)[K], const float (&bs)[K],
                                               int R, int lane, const LnStats& st, float (&y)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) y[i] = K * lane + i < R ? aten_ln_affine<IN_DT>(x[i], wt[i], bs[i], st) : 0.f;
}

// bf16 cache: each channel rounded once (RNE) from the fp32 result.
template <int K>
__device__ __forceinline__ void encode_bf16_lane(const float (&y)[K], uint16_t (&o)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) o[i] = f32_to_bf16(y[i]);
}

// e4m3 per token: y is first rounded to bf16 (the value a bf16 cache would
// hold), amax over the token, scale = max(amax,1e-12)/448, code = RNE(y/scale).
// Padding channels (y = 0) encode as 0.  The token is held by G lanes: the
// wavefront (64) or an aligned group of 16.
template <int K, int G = 64>
__device__ __forceinline__ void encode_e4m3_lane(const float (&y)[K], uint8_t (&codes)[K], float& scale) {
  float yb[K];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    yb[i] = bf16_to_f32(f32_to_bf16(y[i]));
    amax = fmaxf(amax, fabsf(yb[i]));
  }
#pragma unroll
  for (int m = 1; m < G; m <<= 1) amax = fmaxf(amax, shfl_xor_f32(amax, m));
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
// rope_pair<1> (every product and sum rounded to bf16) with the roundings
// done by the hardware conversion, two values per instruction; returns the
// rotated pair packed as bf16 (o1 in the low half).  Finite values and
// infinities round exactly as f32_to_bf16 does (a NaN stays a NaN).
__device__ __forceinline__ uint32_t rope_bf16_packed(float x1, float x2, float c, float s) {
#pragma clang fp contract(off)
  const uint32_t p = pack_bf16x2(x1 * c, x2 * s);
  const uint32_t q = pack_bf16x2(x2 * c, x1 * s);
  return pack_bf16x2(u2f(p << 16) - u2f(p & 0xFFFF0000u), u2f(q << 16) + u2f(q & 0xFFFF0000u));
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
constexpr float kLn2 = 0.6931471805599453f;

// Workgroup barrier that orders LDS only: global loads stay in flight across
// it (a full fence would also wait for them).  The release half completes
// this wave's earlier LDS reads and writes before the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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
