// numerics.h — bit-level conversions shared by the gfx950 kernels and the
// host-side test hooks (the same code runs on both, so a CPU test of the hook
// pins what the kernel computes).
//
// bf16 is carried as raw uint16_t bits.  float8 e4m3fn (OCP: bias 7, no inf,
// 0x7F / 0xFF = NaN, max finite 448) is carried as uint8_t codes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#define SW_HD __host__ __device__ __forceinline__

namespace swamla {

SW_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
SW_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

SW_HD float bf16_to_f32(uint16_t b) { return u2f(static_cast<uint32_t>(b) << 16); }

// Round-to-nearest-even fp32 -> bf16; NaN maps to the canonical quiet NaN.
// This is the rounding eager PyTorch applies after every bf16 op.
SW_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

SW_HD float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Max / sum over each aligned group of W lanes of a wavefront (W = 16, 32
// or 64), every lane of the group receiving the result.  Butterflies without
// the LDS crossbar: DPP quad_perm [1,0,3,2] and [2,3,0,1] (lane ^ 1, ^ 2),
// row_half_mirror (lane i of 8 <-> 7 - i: the other quad) and row_mirror
// (i of 16 <-> 15 - i: the other half-row), then the gfx950 row swaps: after
// permlane16_swap(v, v) the pair holds v[l] and v[l ^ 16] in some order,
// after permlane32_swap v[l] and v[l ^ 32], so max and sum are order-free
// and every lane of a group ends with the same bits.  All W lanes of a
// group must be active.
template <int W, bool MAX>
__device__ __forceinline__ float lane_group_reduce(float v) {
  static_assert(W == 16 || W == 32 || W == 64, "lane group width");
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  auto dpp = [](float x, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value,
                                                                 0xf, 0xf, false));
  };
  v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  v = op(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  v = op(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
  if constexpr (W >= 32) {
    const auto p = __builtin_amdgcn_permlane16_swap(f2u(v), f2u(v), false, false);
    v = op(u2f(p[0]), u2f(p[1]));
  }
  if constexpr (W >= 64) {
    const auto p = __builtin_amdgcn_permlane32_swap(f2u(v), f2u(v), false, false);
    v = op(u2f(p[0]), u2f(p[1]));
  }
  return v;
}
template <int W>
__device__ __forceinline__ float lane_group_max(float v) { return lane_group_reduce<W, true>(v); }
template <int W>
__device__ __forceinline__ float lane_group_sum(float v) { return lane_group_reduce<W, false>(v); }

// fp32 -> e4m3fn code, round-to-nearest-even.  |x| > 464 (past the half-way
// point between 448, the largest finite value, and the next step) and NaN/inf
// give NaN (0x7F | sign); 464 itself ties to even (448).  This is how torch's
// float8_e4m3fn cast behaves.
SW_HD uint8_t f32_to_e4m3(float x) {
  uint32_t u = f2u(x);
  uint8_t sign = static_cast<uint8_t>((u >> 24) & 0x80u);
  u &= 0x7FFFFFFFu;
  if (u > 0x43E80000u) return sign | 0x7F;  // > 464.0f, inf, NaN
  if (u < 0x3C800000u) {                     // below 2^-6: subnormal range
    // |x| * 2^9 is exact; RNE to an integer 0..8 (8 is the code of 2^-6).
    float m = __builtin_rintf(u2f(u) * 512.0f);
    return sign | static_cast<uint8_t>(m);
  }
  uint32_t e = (u >> 23) - 127u + 7u;  // 1..15
  uint32_t mant = u & 0x7FFFFFu;
  uint32_t keep = mant >> 20, rem = mant & 0xFFFFFu;
  uint32_t code = (e << 3) | keep;
  if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) code += 1u;
  return sign | static_cast<uint8_t>(code);
}

// e4m3fn code -> fp32 (exact).
SW_HD float e4m3_to_f32(uint8_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
  if (e == 15u && m == 7u) return u2f(s | 0x7FC00000u);
  if (e == 0u) {
    float v = static_cast<float>(m) * (1.0f / 512.0f);
    return s ? -v : v;
  }
  return u2f(s | ((e + 120u) << 23) | (m << 20));
}

// Four e4m3 codes packed in a uint32 -> four bf16 (two uint32 words, element
// 0 in the low half of lo).  Exact: every finite e4m3 value is a bf16 value.
// The code's exponent/mantissa bits are placed as a bf16 with bias 127 and
// rescaled by 2^120 in fp32, which also maps the e4m3 subnormals correctly.
SW_HD void e4m3x4_to_bf16x4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const float k = 1.329227995784916e+36f;  // 2^120
  uint32_t r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t c = (w >> (8 * i)) & 0xFFu;
    uint32_t bits = ((c & 0x80u) << 24) | ((c & 0x7Fu) << 20);
    r[i] = f2u(u2f(bits) * k) >> 16;  // exact product, exact truncation
  }
  lo = r[0] | (r[1] << 16);
  hi = r[2] | (r[3] << 16);
}

}  // namespace swamla
