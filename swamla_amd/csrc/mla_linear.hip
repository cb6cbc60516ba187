// mla_linear.hip — batched small-row linear layers for the decode step.
//
//   Y[b, m, n] = sum_k X[b, m, k] W[b, n, k] (+ bias[b, n]),  bf16 in/out,
//   fp32 accumulation, one rounding of the result (what a bf16 nn.Linear
//   returns).  M <= 128 rows (the query rows of a decode step).
//
// One launch covers the step's projections that surround attention: wq and
// wkv_a as one product over their stacked weights (models/mla.py:281-288,
// :307), the per-head W_uk absorption of the query and the W_uv read-out of
// the latent output (the re-associated einsums of mla.py:427, :433), and wo
// (mla.py:490-495).  These products have M = 32 rows and read 0.6-6.6 MB of
// weights, so they are bound by launch latency and weight streaming, not by
// MFMA throughput: a block owns a 16-column tile of Y for all M rows, its
// waves (four, or eight for long K) split K, and each wave keeps up to eight
// 32-wide K steps of loads in flight before its MFMAs.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mla_args.h"
#include "mla_plan.h"
#include "numerics.h"

namespace swamla {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// 16-byte global load marked non-temporal (weights are streamed once).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}

// K steps of 32 whose loads are issued together: eight for up to 32 rows,
// fewer for more row tiles so the staged operands stay within the registers.
template <int MT>
constexpr int lin_batch() {
  return MT <= 2 ? 8 : (MT <= 4 ? 4 : 2);
}

// Block: 16 output columns [16*blockIdx.x, +16) of batch entry blockIdx.y
// for all M rows (MT tiles of 16 rows).  Wave w of NW reduces K range
// [w*K/NW, (w+1)*K/NW).  MFMA operands: A = X rows (lane: row l%16, k
// 8(l/16)..+8), B = W rows (lane: column l%16, same k); the result lane holds
// rows 4(l/16)+i of column l%16.  Eight waves serve the long products (K >=
// 1024): each wave's loads then fit in one batch and the weight stream of
// a block is twice as wide.
template <int MT, int NW>
__global__ __launch_bounds__(NW * 64) void mla_linear_kernel(LinearArgs a) {
  __shared__ float red[NW][MT][16][17];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int bt = blockIdx.y;
  const int col0 = blockIdx.x * 16;

  const int kw = a.K / NW;  // multiple of 32 (checked by the caller)
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

  constexpr int kLinBatch = lin_batch<MT>();
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

  // Sum the waves' K ranges in a fixed order, add the bias, round once.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[w][mt][4 * g + i][n] = acc[mt][i];
  __syncthreads();
  const int c = threadIdx.x & 15;
  float bias = 0.f;
  if (a.bias) bias = bf16_to_f32(static_cast<const uint16_t*>(a.bias)[bt * a.bias_bs + col0 + c]);
  uint16_t* Y = static_cast<uint16_t*>(a.y) + bt * a.y_bs + col0 + c;
  for (int e = threadIdx.x >> 4; e < MT * 16; e += NW * 4) {  // e = output row
    const int mt = e >> 4, r = e & 15;
    if (e < a.M) {
      float v = red[0][mt][r][c];
#pragma unroll
      for (int k = 1; k < NW; ++k) v += red[k][mt][r][c];
      if (a.bias) v += bias;
      Y[static_cast<int64_t>(e) * a.y_rs] = f32_to_bf16(v);
    }
  }
}


// ---------------------------------------------------------------------------
// Split merge + W_uv read-out.  Block = (ROWS query rows, head h), 4 waves;
// ROWS (2, 4 or 8) keeps the grid near one block per CU.
// The block first issues its W_uv[h] loads (wave w: output tiles w and w+4,
// all R_pad = 64 NB K; W_uv rows hold R_pad values), then merges its rows'
// split partials into bf16 rows in LDS (thread t < 32*ROWS: row t/32,
// channels 8(t%32) + 256k ..+8; one split: the decode kernel's o_lat row),
// then multiplies: y[r, h, d] = sum_c W_uv[h][d][c] x[r][c].
// ---------------------------------------------------------------------------
template <int DV, int ROWS, int NB, int G>
__global__ __launch_bounds__(256) void mla_merge_project_kernel(MergeProjectArgs a) {
  constexpr int R = 64 * NB;  // R: the padded latent width R_pad
  const int H = a.H;          // heads (16 or 32)
  constexpr int kMpXRow = 2 * R + 16;  // LDS bytes per merged row (padded)
  constexpr int kTilesPerWave = DV / 16 / 4;
  static_assert(ROWS == 2 || ROWS == 4 || ROWS == 8, "rows per block");
  __shared__ __attribute__((aligned(16))) uint8_t x_lds[ROWS * kMpXRow];
  // group states of the split merge (8 = groups x rows): M, T and A per channel
  __shared__ float comb_m[8], comb_t[8];
  __shared__ __attribute__((aligned(16))) float comb_a[G > 1 ? G * ROWS * R : 4];
  // XCD-aware block order: workgroups go to the 8 XCDs round-robin by linear
  // id, so id -> (XCD id % 8, slot id / 8) -> head-major index m gives each
  // XCD the blocks of H / 8 whole heads, and each XCD's L2 fetches only those
  // heads' W_uv (instead of every head's: 8 MB of fetches at 16 heads).
  // The grid has H gx blocks, a multiple of 8.
  const int gx = gridDim.x;
  const int id = blockIdx.y * gx + blockIdx.x;
  const int m = (id & 7) * ((H >> 3) * gx) + (id >> 3);
  const int h = m / gx, r0 = (m - h * gx) * ROWS;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;

  // W_uv[h] rows of this wave's output tiles (B operand: lane = output d),
  // issued right behind the wave's split loads.
  uint4 wb[kTilesPerWave][2 * NB];
  auto load_w = [&]() {
#pragma unroll
    for (int j = 0; j < kTilesPerWave; ++j) {
      const int d = 16 * (w + 4 * j) + n;
      const uint16_t* wp = static_cast<const uint16_t*>(a.w) + h * a.w_hs + static_cast<int64_t>(d) * a.w_rs + 8 * g;
#pragma unroll
      for (int s = 0; s < 2 * NB; ++s) wb[j][s] = *reinterpret_cast<const uint4*>(wp + 32 * s);
    }
  };
  // Merge.  The block's threads form 8 / ROWS groups of ROWS * 32 (whole
  // waves), of which the first G merge: group grp takes splits grp, grp + G,
  // grp + 2G, ... of every row (G > 1 when rows may have more than 8 splits,
  // so their loads go out from several waves at once instead of in rounds of
  // 8; with few splits the extra barrier costs more than it saves).  Within
  // a group: thread -> (row rr, 8 channels cc per 256-channel chunk), one row
  // per half-wave.  Each group forms its own state (max M_g, weight sum T_g,
  // weighted sum A_g); with G > 1 the states meet in LDS and group 0 folds
  // them in group order:
  //   o = sum_g e^(M_g - M) A_g / sum_g e^(M_g - M) T_g,  M = max_g M_g.
  static_assert(G >= 1 && G * ROWS <= 8, "merge groups");
  constexpr int kGT = ROWS * 32;
  const int grp = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kGT);  // wave-uniform
  const bool merging = grp < G;
  const int tg = threadIdx.x - grp * kGT;
  const int rr = tg >> 5, cl = tg & 31;
  const bool hi = (tg & 32) != 0;  // this row's lanes are 32 hi .. 32 hi + 31 of the wave
  const int r = r0 + rr;
  const bool live = r < a.n_rows;  // uniform over the half-wave
  const float* lp = a.lse_part + static_cast<int64_t>(r) * a.n_splits * H + h;
  const float* op0 = a.o_part + (static_cast<int64_t>(r) * a.n_splits * H + h) * R;
  float4 v[8][2];
  // this group's splits j0 .. j0 + 7 of its sequence (split grp + G j)
  auto load_group = [&](int j0, int last, int cc) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float* op = op0 + static_cast<int64_t>(min(grp + G * (j0 + k), last)) * H * R + cc;
      v[k][0] = *reinterpret_cast<const float4*>(op);
      v[k][1] = *reinterpret_cast<const float4*>(op + 4);
    }
  };
  // With n_splits > 1 (the partial buffers are then given, [n_rows, n_splits,
  // H, R_pad]) the group's first 8 splits' partial rows and this lane's
  // split's log-sum-exp go out before the row's split count is known; slots
  // past the count may hold stale, even non-finite, values and are dropped by
  // selects below, never multiplied in.  With n_splits == 1 the buffers may
  // be null and are not touched: every row then reads o_lat.  The W_uv loads
  // go out right behind them (the merge waits only for its own loads).
  const bool early = a.n_splits > 1;  // block-uniform
  const int plan = a.plan ? *a.plan : 0;
  const int L = live ? clamped_row_len(a.ad, r, a.cache_b, a.cache_s) : 0;
  float l0 = -INFINITY;
  if (merging && live && early) {
    l0 = lp[min(grp + G * cl, a.n_splits - 1) * H];
    load_group(0, a.n_splits - 1, 8 * cl);
  }
  load_w();
  // at most n_splits (a plan word from another launch cannot send the reads
  // past the row's slots)
  const int ns = live ? min(row_splits(L, a.n_splits, a.min_chunk, plan).ns, a.n_splits) : 0;
  const int nm = merging && ns > grp ? (ns - grp + G - 1) / G : 0;  // this group's splits of the row
  constexpr int kChunks = (R + 255) / 256;
  float M = -INFINITY, tot = 0.f;
  float macc[kChunks][8];
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) macc[c][i] = 0.f;
  if (ns >= 2 && nm > 0) {
    // Statistics as half-wave reductions: lane cl takes the group's splits
    // cl, cl + 32, ...; max and weight sum are butterflies over the row's 32
    // lanes, and each split's weight is formed once, by its lane.
    if (cl >= nm) l0 = -INFINITY;
    M = l0;
    for (int j = cl + 32; j < nm; j += 32) M = fmaxf(M, lp[(grp + G * j) * H]);
    M = lane_group_max<32>(M);
    const float w0 = l0 == -INFINITY ? 0.f : __expf(l0 - M);
    tot = w0;
    for (int j = cl + 32; j < nm; j += 32) {
      const float l = lp[(grp + G * j) * H];
      tot += l == -INFINITY ? 0.f : __expf(l - M);
    }
    tot = lane_group_sum<32>(tot);
    // Weighted sum over the group's splits in order, 8 at a time; split j's
    // weight comes from lane j % 32 of the row's half (readlane of both
    // halves, then a select).  Every lane of the half runs every chunk, so
    // the lanes read are active.
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int cc = 256 * c + 8 * cl;
      const bool on = cc < R;  // false only in a partial last chunk
      float wl = w0;  // weight of split (j0 & ~31) + cl
      for (int j0 = 0; j0 < nm; j0 += 8) {
        if (j0 > 0 || c > 0) {
          if (on) load_group(j0, ns - 1, cc);
          if (j0 > 0 && (j0 & 31) == 0) {
            const float l = j0 + cl < nm ? lp[(grp + G * (j0 + cl)) * H] : -INFINITY;
            wl = l == -INFINITY ? 0.f : __expf(l - M);
          }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int jj = (j0 & 31) + k;
          const float w_lo = u2f(__builtin_amdgcn_readlane(f2u(wl), jj));
          const float w_hi = u2f(__builtin_amdgcn_readlane(f2u(wl), 32 + jj));
          const bool in = j0 + k < nm;
          const float ws = hi ? w_hi : w_lo;
          const float t[8] = {v[k][0].x, v[k][0].y, v[k][0].z, v[k][0].w, v[k][1].x, v[k][1].y, v[k][1].z, v[k][1].w};
#pragma unroll
          for (int i = 0; i < 8; ++i) macc[c][i] = in ? macc[c][i] + ws * t[i] : macc[c][i];
        }
      }
    }
  }
  if constexpr (G > 1) {
    // group states into LDS: per (group, row) M and T, and A per channel
    if (merging && cl == 0) {
      comb_m[grp * ROWS + rr] = M;
      comb_t[grp * ROWS + rr] = tot;
    }
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int cc = 256 * c + 8 * cl;
      if (merging && cc < R) {
        float* dst = comb_a + (grp * ROWS + rr) * R + cc;
        *reinterpret_cast<float4*>(dst) = make_float4(macc[c][0], macc[c][1], macc[c][2], macc[c][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(macc[c][4], macc[c][5], macc[c][6], macc[c][7]);
      }
    }
    __syncthreads();
  }
  if (grp == 0) {
    if (ns == 1) {
      for (int cc = 8 * cl; cc < R; cc += 256)
        *reinterpret_cast<uint4*>(x_lds + rr * kMpXRow + 2 * cc) =
            *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.o_lat) + r * a.ol_rs + h * a.ol_hs + cc);
    } else if (ns == 0) {
      for (int cc = 8 * cl; cc < R; cc += 256)
        *reinterpret_cast<uint4*>(x_lds + rr * kMpXRow + 2 * cc) = make_uint4(0, 0, 0, 0);
    } else {
      float scale[G];  // e^(M_g - M) per group
      float den = tot;
      if constexpr (G > 1) {
        float Mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < G; ++q) Mx = fmaxf(Mx, comb_m[q * ROWS + rr]);
        den = 0.f;
#pragma unroll
        for (int q = 0; q < G; ++q) {
          const float mq = comb_m[q * ROWS + rr];
          scale[q] = mq == -INFINITY ? 0.f : __expf(mq - Mx);
          den += scale[q] * comb_t[q * ROWS + rr];
        }
      }
      const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        const int cc = 256 * c + 8 * cl;
        if (cc < R) {
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = macc[c][i];
          if constexpr (G > 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
            for (int q = 0; q < G; ++q) {
              const float* src = comb_a + (q * ROWS + rr) * R + cc;
              const float4 p0 = *reinterpret_cast<const float4*>(src), p1 = *reinterpret_cast<const float4*>(src + 4);
              const float t[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
              for (int i = 0; i < 8; ++i) o[i] += scale[q] * t[i];
            }
          }
          uint32_t pk[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            pk[i] = f32_to_bf16(o[2 * i] * inv) | (static_cast<uint32_t>(f32_to_bf16(o[2 * i + 1] * inv)) << 16);
          *reinterpret_cast<uint4*>(x_lds + rr * kMpXRow + 2 * cc) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        }
      }
    }
  }
  __syncthreads();

  // y = X . W_uv[h]^T: A = merged rows (lanes of rows 8..15 repeat rows 0..7;
  // their results are dropped), B = W_uv rows.
  f32x4_t acc[kTilesPerWave];
#pragma unroll
  for (int j = 0; j < kTilesPerWave; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint8_t* xa = x_lds + (n & (ROWS - 1)) * kMpXRow + 2 * (8 * g);
#pragma unroll
  for (int s = 0; s < 2 * NB; ++s) {
    const bf16x8_t av = as_bf16x8(*reinterpret_cast<const uint4*>(xa + 2 * (32 * s)));
#pragma unroll
    for (int j = 0; j < kTilesPerWave; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, as_bf16x8(wb[j][s]), acc[j], 0, 0, 0);
  }
  // lane (n, g) holds rows 4g+i of output column 16*tile + n
  if (4 * g < ROWS) {
#pragma unroll
    for (int j = 0; j < kTilesPerWave; ++j) {
      const int d = 16 * (w + 4 * j) + n;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = r0 + 4 * g + i;
        if (4 * g + i < ROWS && r < a.n_rows)
          static_cast<uint16_t*>(a.y)[r * a.y_rs + h * a.y_hs + d] = f32_to_bf16(acc[j][i]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Packed-weight product for the decode step's two large products (the
// stacked input product and wo): Y[m, n] = sum_k X[m, k] W[n, k] (+ bias[n]).
//
// The weight is packed once per weight version (mla_pack_weight) into 1 KB
// tiles P[o][kb][c][r][e] = W[8o + r][64kb + 8c + e]: an "octet" of 8 output
// rows times 64 k.  One 16-byte load per lane reads a whole tile, i.e. eight
// complete 128-byte lines, and lane l = 8c + r holds row r, k chunk c, which
// is directly an MFMA B operand: for mfma_f32_16x16x32_bf16 lane l is column
// j = l % 16 with k group g = l / 16, so column j holds W row j % 8 at k chunk
// 2g + j / 8.  Columns 0..7 therefore see the even k chunks of rows 0..7 and
// columns 8..15 the odd chunks of the same rows; two MFMAs per tile, one with
// X's even chunks and one with its odd chunks as the A operand, give the
// even and odd halves of each output in separate accumulators, added at the
// end.
//
// Block (bx, slab): X rows [MS*slab, +MS) staged once in LDS with whole-line
// loads, and the block's octets [o0, o1) (at most OPB); the 8 waves split K
// (wave w: k blocks [w*KQ, (w+1)*KQ)).  One block per CU: every CU reads X
// once and an equal share of W.  The waves' partial sums meet in LDS and are
// added in a fixed order (even + odd half per wave, waves 0..7), then the
// bias; one rounding to bf16.
// ---------------------------------------------------------------------------
constexpr int kPkWaves = 8;

template <int MS, int KQ, int OPB>
__global__ __launch_bounds__(kPkWaves * 64) void mla_linear_packed_kernel(PackedLinearArgs a, int n_oct, int gx) {
  constexpr int K = kPkWaves * 64 * KQ;
  constexpr int XS = 2 * K + 16;  // LDS row pitch (bytes): 8 rows of a read pass hit distinct banks
  constexpr int MT = MS / 16;
  // Partial-sum row pitch (floats): 16 OPB + 4, so the four row groups of a
  // store (rows 4g + i, lanes 16g .. 16g + 15) start 16 banks apart and the
  // 64 lanes hit 64 distinct banks (a multiple of 64 would put all four
  // groups on the same 16 banks).
  constexpr int RS = 16 * OPB + 4;
  constexpr int kXBytes = MS * XS, kPartBytes = kPkWaves * MS * RS * 4;
  // The partial sums get LDS of their own when both fit in 160 KB (no
  // barrier between the last X read and the first partial store); else they
  // reuse X's.
  constexpr bool kApart = kXBytes + kPartBytes <= 160 * 1024;
  constexpr int kLds = kApart ? kXBytes + kPartBytes : (kXBytes > kPartBytes ? kXBytes : kPartBytes);
  __shared__ __attribute__((aligned(16))) uint8_t xl[kLds];  // X, and the partial sums
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int slab = blockIdx.y;
  const int o0 = static_cast<int>(static_cast<int64_t>(blockIdx.x) * n_oct / gx);
  const int o1 = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * n_oct / gx);
  // Position advance (one workgroup, one relaxed vector atomic per entry, no
  // return value: nothing waits for it inside the launch; the launch's end
  // makes it visible to the next).  Issued ahead of every load, so that no
  // load result is live across its branch.
  if (a.adv != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && static_cast<int>(threadIdx.x) < a.n_adv)
    __hip_atomic_fetch_add(a.adv + threadIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // X rows of the slab, 16 bytes per thread and load (rows past M repeat the
  // last row; their results are dropped).
  constexpr int kRowB = 2 * K;
  constexpr int XPT = MS * kRowB / (kPkWaves * 64 * 16);
  uint4 xv[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int f = (i * kPkWaves * 64 + static_cast<int>(threadIdx.x)) * 16;
    const int row = f / kRowB, col = f - row * kRowB;
    const int srow = min(MS * slab + row, a.M - 1);
    xv[i] = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a.x) + srow * a.x_rs * 2 + col);
  }
  // W tiles of this wave (octets past o1 - 1 repeat the last one; dropped).
  uint4 wv[OPB][KQ];
#pragma unroll
  for (int o = 0; o < OPB; ++o) {
    const int oc = min(o0 + o, o1 - 1);
    const uint16_t* p = static_cast<const uint16_t*>(a.wp) +
                        (static_cast<int64_t>(oc) * (K / 64) + w * KQ) * 512 + 8 * lane;
#pragma unroll
    for (int q = 0; q < KQ; ++q) wv[o][q] = ld_stream16(p + 512 * q);
  }
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    const int f = (i * kPkWaves * 64 + static_cast<int>(threadIdx.x)) * 16;
    const int row = f / kRowB, col = f - row * kRowB;
    *reinterpret_cast<uint4*>(xl + row * XS + col) = xv[i];
  }
  __syncthreads();

  const int j = lane & 15, g = lane >> 4;
  f32x4_t acc[OPB][MT][2];
#pragma unroll
  for (int o = 0; o < OPB; ++o)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[o][mt][0] = acc[o][mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < KQ; ++q) {
    const int kb = w * KQ + q;
    // A: X[16mt + j][64kb + 16g + 8h .. +8], h = 0 (even chunk) / 1 (odd)
    uint4 av[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        av[mt][h] = *reinterpret_cast<const uint4*>(xl + (16 * mt + j) * XS + 2 * (64 * kb + 16 * g + 8 * h));
#pragma unroll
    for (int o = 0; o < OPB; ++o)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          acc[o][mt][h] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[mt][h]), as_bf16x8(wv[o][q]), acc[o][mt][h], 0, 0, 0);
  }
  if constexpr (!kApart) __syncthreads();  // X is no longer read: its LDS takes the partial sums

  // part[w][row][16o + j]: lanes j < 8 keep the even half of output column
  // 8o + j, lanes j >= 8 the odd half of column 8o + j - 8 (D lane layout:
  // column j, rows 4g + i).
  float* part = reinterpret_cast<float*>(xl + (kApart ? kXBytes : 0));
#pragma unroll
  for (int o = 0; o < OPB; ++o)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        part[(w * MS + 16 * mt + 4 * g + i) * RS + 16 * o + j] = j < 8 ? acc[o][mt][0][i] : acc[o][mt][1][i];
  __syncthreads();
  const int nco = 8 * (o1 - o0);
  const uint16_t* bias = static_cast<const uint16_t*>(a.bias);
  for (int e = threadIdx.x; e < MS * nco; e += kPkWaves * 64) {
    const int r = e / nco, c = e - r * nco;
    const int row = MS * slab + r;
    const int sc = 16 * (c >> 3) + (c & 7);
    if (row < a.M) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < kPkWaves; ++k) v += part[(k * MS + r) * RS + sc] + part[(k * MS + r) * RS + sc + 8];
      if (bias) v += bf16_to_f32(bias[8 * o0 + c]);
      static_cast<uint16_t*>(a.y)[row * a.y_rs + 8 * o0 + c] = f32_to_bf16(v);
    }
  }
}

// Packing: thread -> 8 consecutive k of one row (one 16-byte load and store).
__global__ __launch_bounds__(256) void mla_pack_weight_kernel(PackWeightArgs a) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int kc = a.K / 8;
  if (t >= static_cast<int64_t>(a.N) * kc) return;
  const int n = static_cast<int>(t / kc), k = 8 * static_cast<int>(t - static_cast<int64_t>(n) * kc);
  const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.w) + n * a.w_rs + k);
  const int64_t dst = ((static_cast<int64_t>(n >> 3) * (a.K / 64) + (k >> 6)) * 8 + ((k >> 3) & 7)) * 64 + (n & 7) * 8;
  *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.wp) + dst) = v;
}

}  // namespace

template <int NW>
void launch_linear_nw(const LinearArgs& a, dim3 grid, int mt, hipStream_t s) {
  const dim3 block(NW * 64);
  switch (mt) {
    case 1: hipLaunchKernelGGL((mla_linear_kernel<1, NW>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((mla_linear_kernel<2, NW>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((mla_linear_kernel<3, NW>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((mla_linear_kernel<4, NW>), grid, block, 0, s, a); break;
    case 5: case 6: hipLaunchKernelGGL((mla_linear_kernel<6, NW>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((mla_linear_kernel<8, NW>), grid, block, 0, s, a); break;
  }
}

int launch_linear(const LinearArgs& a, int batch, hipStream_t s) {
  if (a.M == 0 || a.N == 0 || batch == 0) return 0;
  const int mt = (a.M + 15) / 16;
  if (mt < 1 || mt > 8) return -1;
  const dim3 grid(a.N / 16, batch);
  // each wave's K range must be a whole number of 32-wide steps
  if (a.K >= 1024 && a.K % 256 == 0) launch_linear_nw<8>(a, grid, mt, s);
  else launch_linear_nw<4>(a, grid, mt, s);  // K is a multiple of 128 (checked by the caller)
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Rows per slab: as many as keep enough blocks for every CU busy while the
// staged X fits the 160 KB of LDS.
int packed_slab_rows(int M, int N, int K) {
  if (K <= 1024 && M > 32) return 64;
  if (K <= 1024 || (K <= 2048 && N / 8 >= 256)) return M > 16 ? 32 : 16;
  return 16;
}

template <int MS, int KQ>
int launch_packed_ms(const PackedLinearArgs& a, int n_oct, int gx, int slabs, hipStream_t s) {
  const int opb = (n_oct + gx - 1) / gx;
  const dim3 grid(gx, slabs), block(kPkWaves * 64);
  switch (opb) {
    case 1: hipLaunchKernelGGL((mla_linear_packed_kernel<MS, KQ, 1>), grid, block, 0, s, a, n_oct, gx); break;
    case 2: hipLaunchKernelGGL((mla_linear_packed_kernel<MS, KQ, 2>), grid, block, 0, s, a, n_oct, gx); break;
    case 3: hipLaunchKernelGGL((mla_linear_packed_kernel<MS, KQ, 3>), grid, block, 0, s, a, n_oct, gx); break;
    case 4: hipLaunchKernelGGL((mla_linear_packed_kernel<MS, KQ, 4>), grid, block, 0, s, a, n_oct, gx); break;
    default: return -1;
  }
  return 0;
}

template <int MS>
int launch_packed_k(const PackedLinearArgs& a, int n_oct, int gx, int slabs, hipStream_t s) {
  switch (a.K) {
    case 512: return launch_packed_ms<MS, 1>(a, n_oct, gx, slabs, s);
    case 1024: return launch_packed_ms<MS, 2>(a, n_oct, gx, slabs, s);
    case 1536: if constexpr (MS <= 32) return launch_packed_ms<MS, 3>(a, n_oct, gx, slabs, s); else return -1;
    case 2048: if constexpr (MS <= 32) return launch_packed_ms<MS, 4>(a, n_oct, gx, slabs, s); else return -1;
    default: return -1;
  }
}

int launch_linear_packed(const PackedLinearArgs& a, hipStream_t s) {
  if (a.M == 0 || a.N == 0) return 0;
  const int MS = packed_slab_rows(a.M, a.N, a.K);
  const int slabs = (a.M + MS - 1) / MS;
  const int n_oct = a.N / 8;
  int gx = (256 + slabs - 1) / slabs;      // about one block per CU
  gx = max(gx, (n_oct + 3) / 4);           // at most four octets per block
  gx = min(gx, n_oct);
  int rc;
  if (MS == 16) rc = launch_packed_k<16>(a, n_oct, gx, slabs, s);
  else if (MS == 32) rc = launch_packed_k<32>(a, n_oct, gx, slabs, s);
  else rc = launch_packed_k<64>(a, n_oct, gx, slabs, s);
  if (rc) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_pack_weight(const PackWeightArgs& a, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(a.N) * (a.K / 8);
  if (n == 0) return 0;
  hipLaunchKernelGGL(mla_pack_weight_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_merge_project(const MergeProjectArgs& a, hipStream_t s) {
  if (a.n_rows == 0) return 0;
  // rows per block: about one (rows, head) block per CU; every block reads
  // its head's whole W_uv slice, so fewer rows mean more re-reads of it
  const int rows = a.n_rows * a.H <= 2 * 256 ? 2 : (a.n_rows * a.H <= 4 * 256 ? 4 : 8);
  const dim3 grid((a.n_rows + rows - 1) / rows, a.H), block(256);
  const int rc = with_nb(a.R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    // more than 8 splits per row: every wave of the block takes a share of them
    const bool many = a.n_splits > 8;
    if (rows == 2 && many) hipLaunchKernelGGL((mla_merge_project_kernel<128, 2, NB, 4>), grid, block, 0, s, a);
    else if (rows == 2) hipLaunchKernelGGL((mla_merge_project_kernel<128, 2, NB, 1>), grid, block, 0, s, a);
    else if (rows == 4 && many) hipLaunchKernelGGL((mla_merge_project_kernel<128, 4, NB, 2>), grid, block, 0, s, a);
    else if (rows == 4) hipLaunchKernelGGL((mla_merge_project_kernel<128, 4, NB, 1>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((mla_merge_project_kernel<128, 8, NB, 1>), grid, block, 0, s, a);
    return 0;
  });
  if (rc != 0) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace swamla
