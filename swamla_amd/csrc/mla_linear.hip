// mla_linear.hip — batched small-row linear layers for the decode step.
//
//   Y[b, m, n] = sum_k X[b, m, k] W[b, n, k] (+ bias[b, n]),  bf16 in/out,
//   fp32 accumulation, one rounding of the result (what a bf16 nn.Linear
//   returns).  M <= 64 rows (the query rows of a decode step).
//
// One launch covers the step's projections that surround attention: wq and
// wkv_a as one product over their stacked weights (models/mla.py:281-288,
// :307), the per-head W_uk absorption of the query and the W_uv read-out of
// the latent output (the re-associated einsums of mla.py:427, :433), and wo
// (mla.py:490-495).  These products have M = 32 rows and read 0.6-6.6 MB of
// weights, so they are bound by launch latency and weight streaming, not by
// MFMA throughput: a block owns a 16-column tile of Y for all M rows, its
// four waves split K, and each wave keeps up to eight 32-wide K steps of
// loads in flight before its MFMAs.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mla_args.h"
#include "numerics.h"

namespace swamla {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

constexpr int kLinWaves = 4;
constexpr int kLinBatch = 8;  // K steps of 32 whose loads are issued together

// Block: 16 output columns [16*blockIdx.x, +16) of batch entry blockIdx.y
// for all M rows (MT tiles of 16 rows).  Wave w reduces K range
// [w*K/4, (w+1)*K/4).  MFMA operands: A = X rows (lane: row l%16, k
// 8(l/16)..+8), B = W rows (lane: column l%16, same k); the result lane holds
// rows 4(l/16)+i of column l%16.
template <int MT>
__global__ __launch_bounds__(kLinWaves * 64) void mla_linear_kernel(LinearArgs a) {
  __shared__ float red[kLinWaves][MT][16][17];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int bt = blockIdx.y;
  const int col0 = blockIdx.x * 16;

  const int kw = a.K / kLinWaves;  // multiple of 32 (checked by the caller)
  const int kbeg = w * kw;
  const uint16_t* X = static_cast<const uint16_t*>(a.x) + bt * a.x_bs;
  const uint16_t* wr =
      static_cast<const uint16_t*>(a.w) + bt * a.w_bs + static_cast<int64_t>(col0 + n) * a.w_rs + kbeg + 8 * g;
  const uint16_t* xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = min(16 * mt + n, a.M - 1);  // rows past M are computed and dropped
    xr[mt] = X + static_cast<int64_t>(row) * a.x_rs + kbeg + 8 * g;
  }

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int steps = kw / 32;
  for (int s0 = 0; s0 < steps; s0 += kLinBatch) {
    const int cnt = min(kLinBatch, steps - s0);  // block-uniform
    uint4 bv[kLinBatch], av[kLinBatch][MT];
#pragma unroll
    for (int s = 0; s < kLinBatch; ++s) {
      if (s < cnt) {
        bv[s] = *reinterpret_cast<const uint4*>(wr + 32 * (s0 + s));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) av[s][mt] = *reinterpret_cast<const uint4*>(xr[mt] + 32 * (s0 + s));
      }
    }
#pragma unroll
    for (int s = 0; s < kLinBatch; ++s) {
      if (s < cnt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[s][mt]), as_bf16x8(bv[s]), acc[mt], 0, 0, 0);
      }
    }
  }

  // Sum the four waves' K ranges in a fixed order, add the bias, round once.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[w][mt][4 * g + i][n] = acc[mt][i];
  __syncthreads();
  const int r = threadIdx.x >> 4, c = threadIdx.x & 15;
  float bias = 0.f;
  if (a.bias) bias = bf16_to_f32(static_cast<const uint16_t*>(a.bias)[bt * a.bias_bs + col0 + c]);
  uint16_t* Y = static_cast<uint16_t*>(a.y) + bt * a.y_bs + col0 + c;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = 16 * mt + r;
    if (row < a.M) {
      float v = ((red[0][mt][r][c] + red[1][mt][r][c]) + red[2][mt][r][c]) + red[3][mt][r][c];
      if (a.bias) v += bias;
      Y[static_cast<int64_t>(row) * a.y_rs] = f32_to_bf16(v);
    }
  }
}

}  // namespace

int launch_linear(const LinearArgs& a, int batch, hipStream_t s) {
  if (a.M == 0 || a.N == 0 || batch == 0) return 0;
  const dim3 grid(a.N / 16, batch), block(kLinWaves * 64);
  const int mt = (a.M + 15) / 16;
  if (mt == 1) hipLaunchKernelGGL((mla_linear_kernel<1>), grid, block, 0, s, a);
  else if (mt == 2) hipLaunchKernelGGL((mla_linear_kernel<2>), grid, block, 0, s, a);
  else if (mt == 3) hipLaunchKernelGGL((mla_linear_kernel<3>), grid, block, 0, s, a);
  else if (mt == 4) hipLaunchKernelGGL((mla_linear_kernel<4>), grid, block, 0, s, a);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace swamla
