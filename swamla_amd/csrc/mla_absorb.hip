// mla_absorb.hip — per-head products of the prompt pass (prefill-side
// absorption), for row counts past the decode step's:
//
//   y[m, h, n] = sum_k x[m, h, k] w[h, n, k]     bf16 in and out, fp32
//                                                 accumulation, one rounding
//
// The module runs the two re-associated einsums of models/mla.py's absorb
// branch through it (mla.py:427 and :433 up-project the cache; the absorbed
// form moves W_uk onto the queries and W_uv onto the attention output):
//   q_abs[m, h, :] = W_uk[h]^T q_nope[m, h, :]   x = the wq output read in
//       place (row stride H * 192, head stride 192), K = qk_nope_head_dim,
//       N = R_pad, y = q_abs [M, H, R_pad] as the attention kernels read it;
//   o[m, h, :] = W_uv[h] o_lat[m, h, :]          x = o_lat [M, H, R_pad],
//       K = R_pad, N = v_head_dim, y = [M, H * Dv], wo's input layout.
// Both read the strided operands where they lie: no transposes.
//
// Roofline: HBM.  Per row and head the kernel reads K and writes N bf16
// values (2 (K + N) bytes) for 2 K N flops: 85 flop/B at K = 128, N = 256,
// against a bf16 MFMA ridge near 300 flop/B.
//
// Schedule.  One block per CU walks the row tiles of one head h and one
// column tile [z NT, (z + 1) NT) of y (tiles blockIdx.x, + gridDim.x, ...).
// Wave 4 is the loader: it streams x tiles of ROWS rows into a ring of LDS
// buffers (global_load_lds, 48-64 KB ahead) and, once tile i has landed,
// meets the four compute waves at one barrier per tile.  The loader issues
// no stores and the compute waves no loads after their prologue, so each
// wave's vmcnt counts one kind of operation; every tile, the last partial one
// included, issues the same number of DMAs, so the loader's count-based waits
// are exact.
// Compute wave w keeps the W rows of its 16 NBK columns for all K in
// registers for the whole walk.  MFMA (16x16x32 bf16): A = W rows (lane l:
// row l % 16, k 8 (l / 16) .. + 8), B = x rows read from LDS (lane l: row
// l % 16, same k); the result lane holds columns 4 (l / 16) .. + 4 of row
// l % 16, stored as one 8-byte write.
//
// LDS tile: row r at pitch PITCH = K rounded up to 128 values (a multiple of
// 256 bytes); its 16-byte chunk c sits in slot (c & ~15) | ((c ^ r) & 15),
// so the 16 rows of one operand read hit 16 distinct 4-bank groups (gfx950:
// 64 banks of 4 bytes; a 16-byte read serves 16 lanes per cycle).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "mla_args.h"
#include "mla_device.h"
#include "numerics.h"

namespace swamla {
namespace {

typedef __bf16 hb_bf16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned int hb_u32x4_t __attribute__((ext_vector_type(4)));

// Geometry of one instantiation, from KS = K / 32 (K a multiple of 64 up to
// 512).
template <int KS>
struct HpGeo {
  static constexpr int kK = 32 * KS;
  static constexpr int kPitch = (kK + 127) / 128 * 128;  // values per LDS row
  static constexpr int kChunks = kPitch / 8;             // 16-byte slots per LDS row
  static constexpr int kRows = kPitch <= 256 ? 64 : 32;  // a tile is 16-32 KB
  static constexpr int kTileBytes = kRows * kPitch * 2;
  static constexpr int kDma = kTileBytes / 1024;  // the loader's 1 KB DMAs per tile
  // ring depth: the loader keeps 48-64 KB in flight per CU
  static constexpr int kBufs = kTileBytes <= 16384 ? 5 : 3;
  static constexpr int kNbk = KS <= 4 ? 4 : 2;    // 16-column blocks per compute wave
  static constexpr int kNt = 4 * 16 * kNbk;       // columns per block
  static constexpr int kRb = kRows / 16;          // 16-row blocks per tile
  static_assert(KS % 2 == 0 && KS >= 2 && KS <= 16, "K = 64 .. 512, a multiple of 64");
  static_assert(kTileBytes % 1024 == 0 && (kBufs - 2) * kDma < 64, "whole DMAs; vmcnt counts up to 63");
  static_assert(kBufs * kTileBytes <= 160 * 1024, "LDS budget");
};

// 16 bytes per lane from global memory into LDS at dst + 16 * lane
// (non-temporal: x is streamed once).
__device__ __forceinline__ void hp_dma16(const void* src, lds_u8* dst) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<__attribute__((address_space(3))) void*>(dst), 16, 0, 2);
}

// Operand reads of a tile are inline assembly: the compiler cannot tell an
// LDS read of one ring buffer from the DMA still filling another and would
// drain the loads in flight before each read.  Results are released after
// one s_waitcnt lgkmcnt(0).
__device__ __forceinline__ hb_u32x4_t hp_ds_read16(uint32_t addr) {
  hb_u32x4_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

template <int N>
__device__ __forceinline__ void hp_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until at most `ahead` tiles of V DMAs each are in flight.
template <int V, int NBUF>
__device__ __forceinline__ void hp_wait_tiles(int ahead) {
  static_assert(NBUF <= 5, "extend the cases");
  if constexpr (NBUF > 4) if (ahead >= 3) { hp_wait_vm<3 * V>(); return; }
  if constexpr (NBUF > 3) if (ahead >= 2) { hp_wait_vm<2 * V>(); return; }
  if (ahead >= 1) { hp_wait_vm<V>(); return; }
  hp_wait_vm<0>();
}

template <int KS>
__global__ __launch_bounds__(320) void mla_head_product_kernel(HeadProductArgs a) {
  using G = HpGeo<KS>;
  constexpr int K = G::kK, NBK = G::kNbk, RB = G::kRb, ROWS = G::kRows, NBUF = G::kBufs;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NBUF * G::kTileBytes];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = blockIdx.y;
  const int n_tiles = (a.M + ROWS - 1) / ROWS;
  const int stride = gridDim.x;
  const int t0 = blockIdx.x;
  if (t0 >= n_tiles) return;  // uniform per block
  const int my_n = (n_tiles - t0 + stride - 1) / stride;  // tiles t0, t0 + stride, ...
  lds_u8* const ring_p = (lds_u8*)(ring);  // the LDS address space, for the DMA

  if (w == 4) {
    // --- loader.  Tile i of this block goes to buffer i % NBUF.  The DMA of
    // LDS slot p = 64 q + lane (q = 0 .. kDma - 1): row r = p / kChunks,
    // slot s = p % kChunks, which holds chunk c = (s & ~15) | ((s ^ r) & 15).
    // Every tile issues exactly kDma DMAs, which the count-based waits below
    // rely on: rows past M re-read row M - 1 (in bounds; their results are
    // never stored), and only lanes whose chunk lies in the row's padding
    // load nothing — at most half of a row, so no DMA loses all 64 lanes
    // (an instruction whose lanes are all masked off would be branched over
    // and never counted).
    const uint16_t* X = static_cast<const uint16_t*>(a.x) + h * a.x_hs;
    const int64_t last_row = static_cast<int64_t>(a.M) - 1;
    auto issue = [&](int i) {
      const int64_t row0 = static_cast<int64_t>(t0 + i * stride) * ROWS;
      lds_u8* dst = ring_p + (i % NBUF) * G::kTileBytes;
#pragma unroll
      for (int q = 0; q < G::kDma; ++q) {
        const int p = 64 * q + lane;
        const int r = p / G::kChunks, s = p % G::kChunks;
        const int c = (s & ~15) | ((s ^ r) & 15);
        const int64_t row = row0 + r < last_row ? row0 + r : last_row;
        if (c < K / 8) hp_dma16(X + row * a.x_rs + 8 * c, dst + 1024 * q);
      }
    };
    for (int i = 0; i < NBUF - 1 && i < my_n; ++i) issue(i);
    for (int i = 0; i < my_n; ++i) {
      // tile i has landed once at most the DMAs of the tiles after it are in flight
      const int ahead = my_n - 1 - i;
      hp_wait_tiles<G::kDma, NBUF>(ahead < NBUF - 2 ? ahead : NBUF - 2);
      __builtin_amdgcn_s_barrier();
      // every compute wave is past tile i - 1: its buffer takes tile i + NBUF - 1
      if (i + NBUF - 1 < my_n) issue(i + NBUF - 1);
    }
    return;
  }

  // --- compute wave w: columns [col0, col0 + 16 NBK) of y.  Its W rows:
  // column block nb, k step s (lane: row col0 + 16 nb + j, k 32 s + 8 g
  // .. + 8); blocks past N read zeros and are never stored.
  const int col0 = blockIdx.z * G::kNt + w * 16 * NBK;
  const int j = lane & 15, g = lane >> 4;
  const uint16_t* W = static_cast<const uint16_t*>(a.w) + h * a.w_hs;
  uint16_t* Y = static_cast<uint16_t*>(a.y) + h * a.y_hs;
  hb_u32x4_t wf[NBK][KS];
#pragma unroll
  for (int nb = 0; nb < NBK; ++nb) {
    const int n = col0 + 16 * nb + j;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      wf[nb][s] = n < a.N ? *reinterpret_cast<const hb_u32x4_t*>(W + static_cast<int64_t>(n) * a.w_rs + 32 * s + 8 * g)
                          : hb_u32x4_t{0u, 0u, 0u, 0u};
  }
  hp_wait_vm<0>();  // from here on this wave's vmcnt counts only its stores

  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring_p));
  for (int i = 0; i < my_n; ++i) {
    __builtin_amdgcn_s_barrier();  // tile i is in buffer i % NBUF
    f32x4_t acc[NBK][RB];
#pragma unroll
    for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[nb][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const uint32_t tb = lds0 + (i % NBUF) * G::kTileBytes;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      // lane: row 16 rb + j, chunk 4 s + g
      hb_u32x4_t xf[RB];
      const int c = 4 * s + g;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int r = 16 * rb + j;
        const int slot = (c & ~15) | ((c ^ r) & 15);
        xf[rb] = hp_ds_read16(tb + (r * G::kChunks + slot) * 16);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) asm volatile("" : "+v"(xf[rb]));
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[nb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(hb_bf16x8_t, wf[nb][s]),
                                                               __builtin_bit_cast(hb_bf16x8_t, xf[rb]),
                                                               acc[nb][rb], 0, 0, 0);
    }

    // result lane: A rows 4 g .. 4 g + 3 are columns col0 + 16 nb + 4 g + e;
    // its B column j is tile row 16 rb + j
    // (one round-to-nearest-even conversion per value)
    const int64_t row0 = static_cast<int64_t>(t0 + i * stride) * ROWS;
    const bool full = row0 + ROWS <= a.M;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int64_t row = row0 + 16 * rb + j;
      if (!full && row >= a.M) continue;
      uint16_t* yr = Y + row * a.y_rs;
#pragma unroll
      for (int nb = 0; nb < NBK; ++nb) {
        const int n = col0 + 16 * nb + 4 * g;
        if (n < a.N)
          *reinterpret_cast<uint2*>(yr + n) = make_uint2(pack_bf16x2(acc[nb][rb][0], acc[nb][rb][1]),
                                                         pack_bf16x2(acc[nb][rb][2], acc[nb][rb][3]));
      }
    }
  }
}

// f(std::integral_constant<int, KS>) for the built KS = K / 32; -1 if none.
template <typename F>
int with_head_product_ks(int ks, F&& f) {
  switch (ks) {
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 6: return f(std::integral_constant<int, 6>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 10: return f(std::integral_constant<int, 10>{});
    case 12: return f(std::integral_constant<int, 12>{});
    case 14: return f(std::integral_constant<int, 14>{});
    case 16: return f(std::integral_constant<int, 16>{});
    default: return -1;
  }
}

}  // namespace

int launch_head_product(const HeadProductArgs& a, int H, int n_cus, hipStream_t s) {
  if (a.M == 0 || a.N == 0 || H == 0) return 0;
  const int ks = a.K / 32;
  return with_head_product_ks(ks, [&](auto kst) {
    constexpr int KS = decltype(kst)::value;
    using G = HpGeo<KS>;
    const int n_tiles = (a.M + G::kRows - 1) / G::kRows;
    const int nz = (a.N + G::kNt - 1) / G::kNt;
    // about one block per CU over all heads and column tiles
    int gx = (n_cus + H * nz - 1) / (H * nz);
    gx = gx < 1 ? 1 : (gx > n_tiles ? n_tiles : gx);
    hipLaunchKernelGGL((mla_head_product_kernel<KS>), dim3(gx, H, nz), dim3(320), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
  });
}

}  // namespace swamla
