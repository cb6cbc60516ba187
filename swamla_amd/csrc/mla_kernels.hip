// mla_kernels.hip — gfx950 kernels for the MLA latent-KV-cache hot path.
//
//   mla_append_*      fused kv_norm LayerNorm + RoPE(k_pe) + optional e4m3
//                     quantisation + scatter into the ragged cache
//                     (reference: models/mla.py:307-323, :409-414)
//   mla_decode_mfma   absorbed attention over the latent cache, bf16 MFMA,
//                     split-KV partials (reference: models/mla.py:417-487)
//   mla_decode_f32    the same maths in fp32 on the VALU, for fp32 models
//   mla_merge_kernel  log-sum-exp merge of split-KV partials
// (the prefill kernel is in mla_prefill.hip, shared device code in
// mla_device.h)
//
// Geometry: P = 64 (rope dim), H = 16; kv_lora_rank R up to 512, stored
// padded to R_pad = 64 NB channels (kernels are instantiated per NB).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "mla_args.h"
#include "mla_device.h"
#include "mla_plan.h"
#include "numerics.h"

namespace swamla {

// ---------------------------------------------------------------------------
// Kernel 1: fused append.  One wavefront per token, 4 tokens per block.
// ---------------------------------------------------------------------------
// IN_DT: 0 fp32 / 1 bf16 (model dtype; also k_pe cache dtype).
// C_DT : 0 fp32 / 1 bf16 / 2 e4m3 (latent cache dtype).
// The work of one wavefront: token `tok` of the append.
template <int IN_DT, int C_DT, int NB>
__device__ __forceinline__ void append_token(const AppendArgs& a, int tok, int lane) {
  using E = Elem<IN_DT>;
  using T = typename E::T;
  constexpr int RP = 64 * NB;
  const TokAddr ta = tok_addr(a.ad, tok);
  const int b = ta.b, pos = ta.pos, rp = ta.rope;
  if (b < 0 || b >= a.cache_b || pos < 0 || pos >= a.cache_s || rp < 0 || rp >= a.rope_len) {
    if (lane == 0 && a.err_flag) a.err_flag[0] = 1;
    return;
  }
  const T* row = static_cast<const T*>(a.kv_in) + static_cast<int64_t>(tok) * a.in_rs;
  const T* w = static_cast<const T*>(a.ln_w);
  const T* bb = static_cast<const T*>(a.ln_b);

  // --- LayerNorm over c[0..R) in ATen's CPU order: statistics from the whole
  // row, then the affine with lane owning channels NB*lane .. NB*lane+NB-1 of
  // the R_pad-channel input row and LayerNorm parameters (entries >= R unused).
  const LnStats st = aten_ln_stats<IN_DT>(row, a.R, a.eps, lane);
  float x[NB], wt[NB], bs[NB], y[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    x[i] = E::ld(row, NB * lane + i);
    wt[i] = E::ld(w, NB * lane + i);
    bs[i] = E::ld(bb, NB * lane + i);
  }
  layernorm_lane<IN_DT, NB>(x, wt, bs, a.R, lane, st, y);

  const int64_t crow = static_cast<int64_t>(b) * a.cache_s + pos;
  if constexpr (C_DT == 0) {
    uint32_t o[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) o[i] = f2u(y[i]);
    store_lane<NB>(static_cast<uint32_t*>(a.ckv) + crow * RP + NB * lane, o);
  } else if constexpr (C_DT == 1) {
    uint16_t o[NB];
    encode_bf16_lane<NB>(y, o);
    store_lane<NB>(static_cast<uint16_t*>(a.ckv) + crow * RP + NB * lane, o);
  } else {
    float scale;
    uint8_t codes[NB];
    encode_e4m3_lane<NB>(y, codes, scale);
    store_lane<NB>(static_cast<uint8_t*>(a.ckv) + crow * RP + NB * lane, codes);
    if (lane == 0) a.ckv_scale[crow] = scale;
  }

  // --- RoPE on k_pe (input channels R_pad ..): lanes 0..31 own pair i = lane.
  if (lane < kP / 2) {
    const T* ct = static_cast<const T*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
    const T* st = static_cast<const T*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
    const float x1 = E::ld(row, RP + 2 * lane), x2 = E::ld(row, RP + 2 * lane + 1);
    float o1, o2;
    rope_pair<IN_DT>(x1, x2, E::ld(ct, lane), E::ld(st, lane), o1, o2);
    T* dst = static_cast<T*>(a.kpe) + crow * kP + 2 * lane;
    dst[0] = E::from_f32(o1);
    dst[1] = E::from_f32(o2);
  }
}

template <int IN_DT, int C_DT, int NB>
__global__ __launch_bounds__(256) void mla_append_kernel(AppendArgs a) {
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= a.n_tok) return;
  append_token<IN_DT, C_DT, NB>(a, tok, threadIdx.x & 63);
}

// ---------------------------------------------------------------------------
// Split-KV merge of one (row, head) by one wavefront; lane owns 4 channels of
// each 256-channel chunk of the R_pad-channel rows.
//   o = sum_s exp(lse_s - M) o_s / sum_s exp(lse_s - M),  M = max_s lse_s
// Splits are consumed 8 at a time with all their loads in flight, merged
// online across chunks (the reference moves with each chunk's maximum).
// ---------------------------------------------------------------------------
constexpr float kLn2 = 0.6931471805599453f;

// Channels c0 .. c0+3 of one (row, head); lse_out (lane 0 of the first chunk
// only) receives the merged log-sum-exp.
template <int DT>
__device__ __forceinline__ void merge_chunk(const float* __restrict__ o_part, const float* __restrict__ lse_part,
                                            int64_t base, int c0, int r, int h, int ns, int rp, void* o_lat,
                                            int64_t o_rs, int64_t o_hs, float* lse_out) {
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
      v[j] = *reinterpret_cast<const float4*>(o_part + pi * rp + c0);
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
    *reinterpret_cast<float4*>(op + c0) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  } else {
    uint16_t* op = static_cast<uint16_t*>(o_lat) + r * o_rs + h * o_hs;
    uint2 pk;
    pk.x = f32_to_bf16(acc.x * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.y * inv)) << 16);
    pk.y = f32_to_bf16(acc.z * inv) | (static_cast<uint32_t>(f32_to_bf16(acc.w * inv)) << 16);
    *reinterpret_cast<uint2*>(op + c0) = pk;
  }
  if (lse_out) lse_out[static_cast<int64_t>(r) * kH + h] = M + __logf(wsum);
}

template <int DT>
__device__ __forceinline__ void merge_head(const float* __restrict__ o_part, const float* __restrict__ lse_part,
                                           int r, int h, int ns, int n_splits, int rp, void* o_lat, int64_t o_rs,
                                           int64_t o_hs, float* lse_out) {
  const int lane = threadIdx.x & 63;
  const int64_t base = static_cast<int64_t>(r) * n_splits * kH + h;  // lse index of split 0
  for (int c0 = 4 * lane; c0 < rp; c0 += 256) merge_chunk<DT>(o_part, lse_part, base, c0, r, h, ns, rp, o_lat,
                                                              o_rs, o_hs, lse_out && c0 == 0 ? lse_out : nullptr);
}


// ---------------------------------------------------------------------------
// Kernel 2: absorbed decode attention, bf16 MFMA (cache bf16 or e4m3).
//
// One block of four wavefronts per (query row, split).  The waves walk the
// split's tokens in lockstep, 64-token tiles, wave w owning tokens
// 16w..16w+15 of each tile, with DEPTH tiles of its global loads in flight
// in registers.  The loads read whole 128-byte lines: one instruction
// covers 8 tokens x 128 B (lane l: token l%8, bytes 16*(l/8) of a segment);
// loading in the MFMA operand layout instead (16 tokens x 64 B per
// instruction) touches twice the lines per instruction and streams ~25 %
// slower.  Per tile:
//   the wave stores its 16 latent rows (as bf16; e4m3 codes are decoded
//       exactly) and rope rows into the block's LDS tile and reads them back
//       in the MFMA operand layout (lane = token, 8 channels)
//   S^T[16 tok x 16 heads] = K[16 tok x 320] . Q^T[320 x 16 heads]
//       10 x mfma_f32_16x16x32_bf16 on its own tokens; Q^T stays in
//       registers for the whole split
//   the four waves' per-head maxima meet in LDS, so every wave applies the
//       same softmax reference (moved lazily, see kLazy), and each wave writes
//       its bf16 weights P into a shared [16 heads x 64 tokens] LDS array
//   O^T[64 ch x 16 heads] += C^T[64 ch x 64 tok] . P^T[64 tok x 16 heads]
//       8 x mfma_f32_16x16x32_bf16 per wave over ITS 64 of the 256 latent
//       channels (channels 64w..64w+63) and all 64 tokens of the tile.  C^T
//       comes from the tile through ds_read_b64_tr_b16: in each 16-lane
//       group, lane i element k is element i%4 of the 8 bytes addressed by
//       lane i/4 + 4k, so lane s points at C[4g + s/4][c + 4(s%4)].
// Each wave thus ends with the final O of its own channels and nothing is
// combined across waves except the per-head sums of the weights.  Rows with
// more than one split write normalised fp32 partials and their log-sum-exp
// for mla_merge.  (Merging inside this kernel — the last block of a row
// combining the others' partials — needs device-scope release fences, which
// write back the whole L2 of an XCD per block on gfx950 and serialised the
// kernel; it is not done.)
//
// LDS rows are padded so that every access pattern above is free of bank
// conflicts beyond its minimum: latent rows 528 B (16 tokens x 16 B at one
// column hit 16 distinct 16-byte slots), rope rows 144 B.
// ---------------------------------------------------------------------------
// ---- Fused one-token append inside the decode kernel (bf16 model).
// Inputs of one token as loaded by one wavefront: lane owns latent channels
// NB*lane .. +NB-1 (of the R_pad-channel input row and LayerNorm parameters)
// and (lanes 0..31) the k_pe pair `lane`; raw bf16 bits.
template <int NB>
struct FusedIn {
  uint16_t x[NB], wt[NB], bs[NB];
  uint32_t pe;
  uint16_t c, s;
};

template <int NB>
__device__ __forceinline__ FusedIn<NB> fused_load(const AppendArgs& a, int tok, int rope, int lane) {
  const uint16_t* row = static_cast<const uint16_t*>(a.kv_in) + static_cast<int64_t>(tok) * a.in_rs;
  const int pl = lane & (kP / 2 - 1);  // lanes 32..63 repeat pairs 0..31 (unused)
  const int64_t tab = static_cast<int64_t>(rope) * (kP / 2) + pl;
  FusedIn<NB> f;
  load_lane<NB>(row + NB * lane, f.x);
  load_lane<NB>(static_cast<const uint16_t*>(a.ln_w) + NB * lane, f.wt);
  load_lane<NB>(static_cast<const uint16_t*>(a.ln_b) + NB * lane, f.bs);
  f.pe = *reinterpret_cast<const uint32_t*>(row + 64 * NB + 2 * pl);
  f.c = static_cast<const uint16_t*>(a.cos_tab)[tab];
  f.s = static_cast<const uint16_t*>(a.sin_tab)[tab];
  return f;
}

// The token in cache form: `row` is the lane's NB latent channels as the
// attention reads them (bf16; for e4m3 the decoded codes), `pe` its rotated
// k_pe pair, plus the e4m3 codes and scale.
template <int C_DT, int NB>
struct FusedTok {
  uint16_t row[NB];
  uint8_t codes[NB];
  uint32_t pe;
  float scale;
};

// Same arithmetic as append_token<1, C_DT, NB>; `row` is the token's wkv_a
// row (the statistics read it in their own order).
template <int C_DT, int NB>
__device__ __forceinline__ FusedTok<C_DT, NB> fused_compute(const FusedIn<NB>& f, const uint16_t* row, float eps,
                                                            int R, int lane) {
  const LnStats st = aten_ln_stats<1>(row, R, eps, lane);
  float x[NB], wt[NB], bs[NB], y[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    x[i] = bf16_to_f32(f.x[i]);
    wt[i] = bf16_to_f32(f.wt[i]);
    bs[i] = bf16_to_f32(f.bs[i]);
  }
  layernorm_lane<1, NB>(x, wt, bs, R, lane, st, y);
  FusedTok<C_DT, NB> t;
  t.scale = 1.f;
  if constexpr (C_DT == 1) {
    encode_bf16_lane<NB>(y, t.row);
  } else {
    encode_e4m3_lane<NB>(y, t.codes, t.scale);
#pragma unroll
    for (int i = 0; i < NB; ++i) t.row[i] = e4m3_to_bf16_bits(t.codes[i]);
  }
  float o1, o2;
  rope_pair<1>(u2f(f.pe << 16), u2f(f.pe & 0xFFFF0000u), u2f(static_cast<uint32_t>(f.c) << 16),
               u2f(static_cast<uint32_t>(f.s) << 16), o1, o2);
  t.pe = f32_to_bf16(o1) | (static_cast<uint32_t>(f32_to_bf16(o2)) << 16);
  return t;
}

template <int C_DT, int NB>
__device__ __forceinline__ void fused_store(const AppendArgs& a, int64_t crow, const FusedTok<C_DT, NB>& t,
                                            int lane) {
  if constexpr (C_DT == 1) {
    store_lane<NB>(static_cast<uint16_t*>(a.ckv) + crow * (64 * NB) + NB * lane, t.row);
  } else {
    store_lane<NB>(static_cast<uint8_t*>(a.ckv) + crow * (64 * NB) + NB * lane, t.codes);
    if (lane == 0) a.ckv_scale[crow] = t.scale;
  }
  if (lane < kP / 2) reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.kpe) + crow * kP)[lane] = t.pe;
}

// Occupancy of the decode kernel by cache type.  A bf16 tile streams at the
// HBM rate with one workgroup per CU (four waves, one per SIMD) and DEPTH 2
// tiles of loads in flight per wave.  An e4m3 tile carries 40% fewer bytes
// through the same LDS/MFMA/softmax chain (plus the e4m3 decode), so with
// one wave per SIMD that chain's latency, not HBM, sets the tile rate; at
// ranks up to 256 three workgroups share a CU instead (one tile of loads in
// flight per wave, at most 168 VGPRs, 3 x 45.7 KB of LDS), and each wave's
// waits hide under the other workgroups' work.  The split plan asks
// mla_decode_blocks_per_cu how many workgroups a CU holds.
template <int C_DT, int NB>
struct DecodeShape {
  static constexpr bool kShared = C_DT == 2 && NB <= 4;
  static constexpr int kDepth = kShared ? 1 : 2;       // tiles of loads in flight per wave
  static constexpr int kWavesPerEU = kShared ? 3 : 1;  // workgroups per CU
};

template <int C_DT, int DEPTH, bool FUSE, int NB>
__global__ __launch_bounds__(kWaves * 64, (DecodeShape<C_DT, NB>::kWavesPerEU)) void mla_decode_mfma(DecodeArgs a) {
  constexpr int RP = LatGeo<NB>::RP, kCRow = LatGeo<NB>::CRow;
  __shared__ __attribute__((aligned(16))) uint8_t c_lds[LatGeo<NB>::CBytes];
  __shared__ __attribute__((aligned(16))) uint8_t pe_lds[kPeBytes];
  __shared__ __attribute__((aligned(16))) uint8_t p_lds[kH * kPRow];
  __shared__ float mx_lds[kWaves][kH];
  __shared__ float l_lds[kWaves][kH];

  // Workgroup -> (row, split): the grid's (x, y), or with a balanced plan the
  // position of blockIdx.x among all rows' splits (every wave computes the
  // same plan; the values are uniform).
  int r = blockIdx.y, split = blockIdx.x, bal_chunk = 0;
  TokAddr ra;
  if (a.balance > 0) {
    const BalancedSlot bs =
        balanced_slot(a.ad, a.n_rows, a.cache_b, a.cache_s, a.n_splits, a.min_chunk, a.balance, blockIdx.x);
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.plan) *a.plan = bs.chunk;
    if (!bs.ok) return;
    r = __builtin_amdgcn_readfirstlane(bs.r);
    split = __builtin_amdgcn_readfirstlane(bs.split);
    bal_chunk = bs.chunk;
    ra = bs.addr;  // no second dependent load of the row's position
  } else {
    ra = row_addr(a.ad, r);
  }
  // The wave index is read into a scalar register so loop control below is
  // uniform (scalar branches, no exec masking) and the compiler can track
  // the in-flight loads across iterations.
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int lt = lane & 7, lc = lane >> 3;  // whole-line loads: token, 16-byte column

  const int b = ra.b;
  int L = ra.pos;
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const RowSplits rsp = row_splits(L, a.n_splits, a.min_chunk, bal_chunk);
  const int ns = rsp.ns;
  if (split >= ns && !(ns == 0 && split == 0)) return;
  const int chunk = rsp.chunk;
  const int t0 = split * chunk;
  const int t1 = min(L, t0 + chunk);
  const int n_tiles = t1 > t0 ? (t1 - t0 + kTileTok - 1) / kTileTok : 0;  // block-uniform

  // Fused one-token append (FUSE): the block owning row r's last split turns
  // the row's wkv_a output into its new cache token (position L - 1, the last
  // token of that split), writes it to the cache at the end, and puts the
  // computed row into LDS in place of the cache row it loaded, so no load of
  // this launch depends on the store.  One wave (the one whose 16 tokens hold
  // position L - 1) does the work; its input loads go out first and the
  // arithmetic runs while the first tiles are in flight.
  bool fa_own = false;  // block-uniform
  int fa_w = 0, fa_k = 0;
  TokAddr fa_t{0, 0, 0};
  if constexpr (FUSE) {
    if (split == (ns > 0 ? ns - 1 : 0)) {
      // fa.ad is the launch's own dense addressing with one row per sequence,
      // so the new token's cache row, position and RoPE row follow from ra.
      fa_t = TokAddr{ra.b, ra.pos - 1, ra.rope};
      if (fa_t.b < 0 || fa_t.b >= a.fa.cache_b || fa_t.pos < 0 || fa_t.pos >= a.fa.cache_s || fa_t.rope < 0 ||
          fa_t.rope >= a.fa.rope_len) {
        if (threadIdx.x == 0 && a.fa.err_flag) a.fa.err_flag[0] = 1;  // skipped, as mla_append does
      } else {
        fa_own = true;  // then L = pos + 1 <= cache_s and t1 = L
        const int tn = fa_t.pos - t0;
        fa_w = (tn & (kTileTok - 1)) >> 4;
        fa_k = tn & (kSub - 1);
      }
    }
  }
  const bool fa_wave = FUSE && fa_own && w == fa_w;  // wave-uniform
  // Every wave of a fused launch issues these loads (valid addresses: its
  // own input row, RoPE row 0 unless it owns the append) so that no value
  // crosses a branch: the loaded registers are consumed only by fa_wave,
  // well after the tile loads behind them have been issued.
  FusedIn<NB> fin;
  if constexpr (FUSE) {
    fin = fused_load<NB>(a.fa, r, fa_own ? fa_t.rope : 0, lane);
    // keep these loads ahead of the tile loads (they are waited for first)
    asm volatile("" ::: "memory");
  }

  // Loads are issued unconditionally, so every address is clamped to a valid
  // cache element: an invalid or empty row reads row 0, token 0.
  const int64_t cache_row0 = static_cast<int64_t>((b < 0 || b >= a.cache_b) ? 0 : b) * a.cache_s;
  const int t_last = t1 > 0 ? t1 - 1 : 0;

  // Global loads of this wave's 16 tokens of tile j (tokens clamped into
  // range; the surplus ones are masked in the softmax).
  auto load_tile = [&](int j, KTile<C_DT, NB>& kt) {
    const int wbase = t0 + j * kTileTok + kSub * w;
    const int64_t row_a = cache_row0 + min(wbase + lt, t_last);
    const int64_t row_b = cache_row0 + min(wbase + 8 + lt, t_last);
    if constexpr (C_DT == 2) {
      const uint8_t* ca = static_cast<const uint8_t*>(a.ckv) + row_a * RP;
      const uint8_t* cb = static_cast<const uint8_t*>(a.ckv) + row_b * RP;
#pragma unroll
      for (int q = 0; q < (NB + 1) / 2; ++q) {
        // for odd NB the last segment is half a row: its upper lanes re-read
        // the first half (in the row, not stored)
        const int col = 128 * q + ((NB & 1) && q == NB / 2 ? 16 * (lc & 3) : 16 * lc);
        kt.c[2 * q] = ld_stream16(ca + col);
        kt.c[2 * q + 1] = ld_stream16(cb + col);
      }
      const int tb = wbase + 4 * g;  // scales of the 4 tokens this lane scores
      const float* sp = a.ckv_scale + cache_row0;
      kt.sc.x = sp[min(tb + 0, t_last)];
      kt.sc.y = sp[min(tb + 1, t_last)];
      kt.sc.z = sp[min(tb + 2, t_last)];
      kt.sc.w = sp[min(tb + 3, t_last)];
    } else {
      const uint8_t* ca = static_cast<const uint8_t*>(a.ckv) + row_a * (2 * RP) + 16 * lc;
      const uint8_t* cb = static_cast<const uint8_t*>(a.ckv) + row_b * (2 * RP) + 16 * lc;
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        kt.c[2 * q] = ld_stream16(ca + 128 * q);
        kt.c[2 * q + 1] = ld_stream16(cb + 128 * q);
      }
    }
    const uint8_t* kpe = static_cast<const uint8_t*>(a.kpe);
    kt.p[0] = ld_stream16(kpe + row_a * (2 * kP) + 16 * lc);
    kt.p[1] = ld_stream16(kpe + row_b * (2 * kP) + 16 * lc);
  };

  // ---- Q^T operand (B of S^T): lane holds head n, channels 32s + 8g..+8.
  KTile<C_DT, NB> kt[DEPTH];
  bf16x8_t qb[2 * NB + 2];
  {
    const uint16_t* qa = static_cast<const uint16_t*>(a.q_abs) + r * a.qa_rs + n * a.qa_hs;
    // channels >= R (the padding of R_pad) are zeroed
#pragma unroll
    for (int s = 0; s < 2 * NB; ++s)
      qb[s] = as_bf16x8(mask_bf16x8(*reinterpret_cast<const uint4*>(qa + 32 * s + 8 * g), a.R - (32 * s + 8 * g)));
    // q_pe with interleaved RoPE at the row's table position
    const uint16_t* qp = static_cast<const uint16_t*>(a.q_pe) + r * a.qp_rs + n * a.qp_hs;
    int rp = ra.rope;
    rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
    const uint16_t* ct = static_cast<const uint16_t*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
    const uint16_t* st = static_cast<const uint16_t*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
    uint4 raw[2];
    uint2 cr[2], sr[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c0 = 32 * s + 8 * g;
      raw[s] = *reinterpret_cast<const uint4*>(qp + c0);
      cr[s] = *reinterpret_cast<const uint2*>(ct + c0 / 2);
      sr[s] = *reinterpret_cast<const uint2*>(st + c0 / 2);
    }
    // Q's loads are issued first, the tiles' right behind them: waiting for
    // Q leaves every tile load in flight.
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load_tile(d, kt[d]);
    // the fused append's arithmetic below must not pull these loads after it
    if constexpr (FUSE) asm volatile("" ::: "memory");
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t wv_in[4] = {raw[s].x, raw[s].y, raw[s].z, raw[s].w};
      const uint32_t cw2[2] = {cr[s].x, cr[s].y}, sw2[2] = {sr[s].x, sr[s].y};
      uint32_t wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t cj = (j & 1) ? (cw2[j >> 1] >> 16) : (cw2[j >> 1] & 0xFFFF);
        const uint32_t sj = (j & 1) ? (sw2[j >> 1] >> 16) : (sw2[j >> 1] & 0xFFFF);
        float o1, o2;
        rope_pair<1>(bf16_to_f32(wv_in[j] & 0xFFFF), bf16_to_f32(wv_in[j] >> 16), bf16_to_f32(cj),
                     bf16_to_f32(sj), o1, o2);
        wv[j] = f32_to_bf16(o1) | (static_cast<uint32_t>(f32_to_bf16(o2)) << 16);
      }
      qb[2 * NB + s] = as_bf16x8(make_uint4(wv[0], wv[1], wv[2], wv[3]));
    }
  }

  // The new token in cache form (fused append), computed while the first
  // tiles load.
  FusedTok<C_DT, NB> ftok;
  if constexpr (FUSE)
    if (fa_wave)
      ftok = fused_compute<C_DT, NB>(
          fin, static_cast<const uint16_t*>(a.fa.kv_in) + static_cast<int64_t>(r) * a.fa.in_rs, a.fa.eps, a.R, lane);

  f32x4_t oacc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  // LDS addresses of this lane.  Stores (whole-line layout): token
  // 16w + lt (+8), column 16*lc of a 128-byte segment.  Operand reads: token
  // 16w + n, 8 channels at 32s + 8g.  C^T reads: token row 4g + n/4 of each
  // 16-token block, channel 16NB w + 4(n%4) (+16 mb).
  uint8_t* const c_st = c_lds + (kSub * w + lt) * kCRow + 16 * lc;
  uint8_t* const pe_st = pe_lds + (kSub * w + lt) * kPeRow + 16 * lc;
  const uint8_t* const c_op = c_lds + (kSub * w + n) * kCRow + 2 * (8 * g);
  const uint8_t* const pe_op = pe_lds + (kSub * w + n) * kPeRow + 2 * (8 * g);
  const uint8_t* const c_tr = c_lds + (4 * g + (n >> 2)) * kCRow + 2 * (16 * NB * w) + 8 * (n & 3);
  uint8_t* const p_mine = p_lds + n * kPRow + 2 * (kSub * w + 4 * g);
  const uint8_t* const p_row = p_lds + n * kPRow + 2 * (4 * g);

  auto process = [&](int j, KTile<C_DT, NB>& kt) {
    const int wbase = t0 + j * kTileTok + kSub * w;
    const bool full = t0 + (j + 1) * kTileTok <= t1;  // block-uniform

    // This wave's latent and rope rows into the tile (e4m3 decoded to bf16).
    if constexpr (C_DT == 2) {
#pragma unroll
      for (int q = 0; q < 2 * ((NB + 1) / 2); ++q) {
        const uint2 a0 = e4m3x4_to_bf16x4_hw(kt.c[q].x), a1 = e4m3x4_to_bf16x4_hw(kt.c[q].y);
        const uint2 a2 = e4m3x4_to_bf16x4_hw(kt.c[q].z), a3 = e4m3x4_to_bf16x4_hw(kt.c[q].w);
        // 16 codes: token 16w + 8(q&1) + lt, channels 128(q>>1) + 16lc..+16
        // (the re-read upper half of an odd NB's last segment is not stored)
        if ((NB & 1) && (q >> 1) == NB / 2 && lc >= 4) continue;
        uint8_t* dst = c_lds + (kSub * w + 8 * (q & 1) + lt) * kCRow + 2 * (128 * (q >> 1) + 16 * lc);
        *reinterpret_cast<uint4*>(dst) = make_uint4(a0.x, a0.y, a1.x, a1.y);
        *reinterpret_cast<uint4*>(dst + 16) = make_uint4(a2.x, a2.y, a3.x, a3.y);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 2 * NB; ++s) {
        // element-wise: a whole-struct copy becomes a memcpy that keeps kt
        // out of registers
        const uint4 v = kt.c[s];
        *reinterpret_cast<uint4*>(c_st + 8 * (s & 1) * kCRow + 128 * (s >> 1)) = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
    *reinterpret_cast<uint4*>(pe_st) = kt.p[0];
    *reinterpret_cast<uint4*>(pe_st + 8 * kPeRow) = kt.p[1];
    float4 scv = make_float4(1.f, 1.f, 1.f, 1.f);
    if constexpr (C_DT == 2) scv = kt.sc;
    if constexpr (FUSE) {
      if (fa_wave && j == n_tiles - 1) {
        // The new token's row: the computed values replace what was loaded
        // (this wave's own rows, so its reads below see them in order).
        store_lane<NB>(reinterpret_cast<uint16_t*>(c_lds + (kSub * w + fa_k) * kCRow) + NB * lane, ftok.row);
        if (lane < kP / 2) *reinterpret_cast<uint32_t*>(pe_lds + (kSub * w + fa_k) * kPeRow + 4 * lane) = ftok.pe;
        if constexpr (C_DT == 2) {
          if (g == (fa_k >> 2)) {
            const int i = fa_k & 3;
            scv.x = i == 0 ? ftok.scale : scv.x;
            scv.y = i == 1 ? ftok.scale : scv.y;
            scv.z = i == 2 ? ftok.scale : scv.z;
            scv.w = i == 3 ? ftok.scale : scv.w;
          }
        }
      }
    }

    // The registers of kt are free: refill them with the tile DEPTH ahead
    // (unconditionally, see above).
    load_tile(j + DEPTH, kt);

    // S^T = K . Q^T from the wave's own rows (LDS operations of one wave
    // complete in order, so no wait beyond the operand reads is needed).
    f32x4_t s_c = {0.f, 0.f, 0.f, 0.f}, s_p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2 * NB; ++s)
      s_c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          as_bf16x8(*reinterpret_cast<const uint4*>(c_op + 2 * (32 * s))), qb[s], s_c, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < 2; ++s)
      s_p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          as_bf16x8(*reinterpret_cast<const uint4*>(pe_op + 2 * (32 * s))), qb[2 * NB + s], s_p, 0, 0, 0);

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
        if (wbase + 4 * g + i >= t1) x[i] = -INFINITY;
    }
    float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mt = wave_max_rows(mt);  // max over this wave's 16 tokens of head n
    if (g == 0) mx_lds[w][n] = mt;
    lds_barrier();  // latent rows and maxima of all waves are visible

    // C^T of this wave's channels for the whole tile; the reads' latency
    // hides under the softmax below.
    s16x4_t ct[2][NB][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int mb = 0; mb < NB; ++mb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          ct[kb][mb][h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4_t*)(c_tr + (32 * kb + 16 * h) * kCRow + 32 * mb));

    // Online softmax in the log2 domain with a lazily moved reference shared
    // by the four waves: m_run only moves when a head's tile maximum exceeds
    // it by more than kLazy, so weights stay <= 2^kLazy and O is rescaled
    // rarely (the normalisation by l is exact either way).  Every wave sees
    // the same maxima, so the branch is taken alike in all four.
    const float mtile = fmaxf(fmaxf(mx_lds[0][n], mx_lds[1][n]), fmaxf(mx_lds[2][n], mx_lds[3][n]));
    if (__any(mtile > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, mtile);  // finite: the tile's first token is valid
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
#pragma unroll
      for (int mb = 0; mb < NB; ++mb) oacc[mb] = oacc[mb] * alpha;
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
    *reinterpret_cast<uint2*>(p_mine) = pw;
    // P of all waves is visible; every wave's reads of this tile's rows have
    // completed, so the next tile may overwrite them.
    lds_barrier();

    // O^T[16NB w + 16mb + ., head] += C^T . P^T over the tile's two 32-token
    // halves; the 8 K slots of lane group g are tokens 32kb + 4g + {0..3}
    // and 32kb + 16 + 4g + {0..3} in both operands.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const uint2 plo = *reinterpret_cast<const uint2*>(p_row + 2 * (32 * kb));
      const uint2 phi = *reinterpret_cast<const uint2*>(p_row + 2 * (32 * kb + 16));
      const bf16x8_t pb = as_bf16x8(make_uint4(plo.x, plo.y, phi.x, phi.y));
#pragma unroll
      for (int mb = 0; mb < NB; ++mb)
        oacc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cat_bf16x8(ct[kb][mb][0], ct[kb][mb][1]), pb,
                                                           oacc[mb], 0, 0, 0);
    }
  };

  // Full groups of DEPTH tiles in the loop, the remainder after it; every
  // branch is block-uniform.  Surplus refills at the end of the stream
  // re-read the split's last row (cache hits) and drain in order right
  // behind the real tiles.
  int it = 0;
  for (; it + DEPTH <= n_tiles; it += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) process(it + d, kt[d]);
  }
#pragma unroll
  for (int d = 0; d < DEPTH - 1; ++d)
    if (it + d < n_tiles) process(it + d, kt[d]);

  if constexpr (FUSE)
    if (fa_wave) fused_store<C_DT, NB>(a.fa, static_cast<int64_t>(fa_t.b) * a.fa.cache_s + fa_t.pos, ftok, lane);

  // ---- Sum of the weights per head over the four waves.
  float l_w = l_part + shfl_xor_f32(l_part, 16);
  l_w += shfl_xor_f32(l_w, 32);
  if (g == 0) l_lds[w][n] = l_w;
  lds_barrier();
  const float Ltot = (l_lds[0][n] + l_lds[1][n]) + (l_lds[2][n] + l_lds[3][n]);
  const float inv = Ltot > 0.f ? 1.f / Ltot : 0.f;

  // Lane (n, g) holds head n, channels 16NB w + 16mb + 4g + {0..3} (the
  // padding channels come out as 0: their cache channels hold 0).
  const int ch0 = 16 * NB * w + 4 * g;
  if (ns <= 1) {
    uint16_t* op = static_cast<uint16_t*>(a.o_lat) + r * a.o_rs + n * a.o_hs + ch0;
#pragma unroll
    for (int mb = 0; mb < NB; ++mb) {
      uint2 pk;
      pk.x = f32_to_bf16(oacc[mb][0] * inv) | (static_cast<uint32_t>(f32_to_bf16(oacc[mb][1] * inv)) << 16);
      pk.y = f32_to_bf16(oacc[mb][2] * inv) | (static_cast<uint32_t>(f32_to_bf16(oacc[mb][3] * inv)) << 16);
      *reinterpret_cast<uint2*>(op + 16 * mb) = pk;
    }
    return;
  }
  const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + n;
  float* op = a.o_part + pidx * RP + ch0;
#pragma unroll
  for (int mb = 0; mb < NB; ++mb)
    *reinterpret_cast<float4*>(op + 16 * mb) =
        make_float4(oacc[mb][0] * inv, oacc[mb][1] * inv, oacc[mb][2] * inv, oacc[mb][3] * inv);
  if (w == 0 && g == 0) a.lse_part[pidx] = (Ltot > 0.f) ? (m_run + __log2f(Ltot)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Kernel 2 (fp32 models): the same maths on the VALU in fp32.  One block of
// 256 threads per (row, split); 16-token tiles staged in LDS.
// ---------------------------------------------------------------------------
template <int NB>
__global__ __launch_bounds__(256) void mla_decode_f32(DecodeArgs a) {
  constexpr int TT = 16;
  constexpr int RP = 64 * NB, KC = RP + kP;  // channels scored per cached token
  constexpr int CPV = RP / 16;               // output channels per thread
  __shared__ float q_s[kH][KC + 1];
  __shared__ float k_s[TT][KC + 1];
  __shared__ float p_s[kH][TT];
  __shared__ float alpha_s[kH];
  __shared__ float m_s[kH], l_s[kH];

  int r = blockIdx.y, split = blockIdx.x, bal_chunk = 0;
  const int t = threadIdx.x;
  TokAddr ra;
  if (a.balance > 0) {  // as in mla_decode_mfma
    const BalancedSlot bs =
        balanced_slot(a.ad, a.n_rows, a.cache_b, a.cache_s, a.n_splits, a.min_chunk, a.balance, blockIdx.x);
    if (blockIdx.x == 0 && t == 0 && a.plan) *a.plan = bs.chunk;
    if (!bs.ok) return;
    r = __builtin_amdgcn_readfirstlane(bs.r);
    split = __builtin_amdgcn_readfirstlane(bs.split);
    bal_chunk = bs.chunk;
    ra = bs.addr;
  } else {
    ra = row_addr(a.ad, r);
  }
  const int b = ra.b;
  int L = ra.pos;
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const RowSplits rsp = row_splits(L, a.n_splits, a.min_chunk, bal_chunk);
  const int ns = rsp.ns;
  if (split >= ns && !(ns == 0 && split == 0)) return;
  const int chunk = rsp.chunk;
  const int t0 = split * chunk, t1 = min(L, t0 + chunk);
  const int64_t row0 = static_cast<int64_t>(b < 0 ? 0 : b) * a.cache_s;

  int rp = ra.rope;
  rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
  const float* qa = static_cast<const float*>(a.q_abs) + r * a.qa_rs;
  const float* qp = static_cast<const float*>(a.q_pe) + r * a.qp_rs;
  const float* ct = static_cast<const float*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
  const float* st = static_cast<const float*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
  for (int i = t; i < kH * RP; i += 256) {
    const int h = i / RP, c = i % RP;
    q_s[h][c] = c < a.R ? qa[h * a.qa_hs + c] : 0.f;  // the padding channels are zero
  }
  for (int i = t; i < kH * kP / 2; i += 256) {
    const int h = i / (kP / 2), pi = i % (kP / 2);
    float o1, o2;
    rope_pair<0>(qp[h * a.qp_hs + 2 * pi], qp[h * a.qp_hs + 2 * pi + 1], ct[pi], st[pi], o1, o2);
    q_s[h][RP + 2 * pi] = o1;
    q_s[h][RP + 2 * pi + 1] = o2;
  }
  if (t < kH) {
    m_s[t] = -INFINITY;
    l_s[t] = 0.f;
  }
  const int h_pv = t >> 4, c_pv = (t & 15) * CPV;
  float o[CPV];
#pragma unroll
  for (int j = 0; j < CPV; ++j) o[j] = 0.f;

  const float* ckv = static_cast<const float*>(a.ckv);
  const float* kpe = static_cast<const float*>(a.kpe);
  for (int base = t0; base < t1; base += TT) {
    __syncthreads();
    for (int i = t; i < TT * KC; i += 256) {
      const int j = i / KC, c = i % KC;
      const int tok = base + j;
      float v = 0.f;
      if (tok < t1) v = c < RP ? ckv[(row0 + tok) * RP + c] : kpe[(row0 + tok) * kP + (c - RP)];
      k_s[j][c] = v;
    }
    __syncthreads();
    {  // scores: thread -> head t/16, token t%16
      const int h = t >> 4, j = t & 15;
      float acc = 0.f;
      for (int c = 0; c < KC; ++c) acc += q_s[h][c] * k_s[j][c];
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
    for (int jj = 0; jj < CPV; ++jj) o[jj] *= al;
    for (int j = 0; j < TT; ++j) {
      const float p = p_s[h_pv][j];
#pragma unroll
      for (int jj = 0; jj < CPV; ++jj) o[jj] += p * k_s[j][c_pv + jj];
    }
  }
  __syncthreads();
  const float Lh = l_s[h_pv];
  const float inv = Lh > 0.f ? 1.f / Lh : 0.f;
  if (ns <= 1) {
    float* op = static_cast<float*>(a.o_lat) + r * a.o_rs + h_pv * a.o_hs + c_pv;
#pragma unroll
    for (int jj = 0; jj < CPV; ++jj) op[jj] = o[jj] * inv;
    return;
  }
  const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + h_pv;
  float* op = a.o_part + pidx * RP + c_pv;
#pragma unroll
  for (int jj = 0; jj < CPV; ++jj) op[jj] = o[jj] * inv;
  if ((t & 15) == 0) a.lse_part[pidx] = (Lh > 0.f) ? (m_s[h_pv] + __log2f(Lh)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Kernel 3: split-KV merge, one wavefront per (row, head).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(64) void mla_merge_kernel(MergeArgs a) {
  const int h = blockIdx.x, r = blockIdx.y;
  const int ns = row_splits(clamped_row_len(a.ad, r, a.cache_b, a.cache_s), a.n_splits, a.min_chunk,
                            a.plan ? *a.plan : 0).ns;
  if (ns <= 1) return;  // written by the decode kernel
  merge_head<DT>(a.o_part, a.lse_part, r, h, ns, a.n_splits, 64 * ((a.R + 63) / 64), a.o_lat, a.o_rs, a.o_hs,
                 a.lse_out);
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
  const int rc = with_nb(a.R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    if (in_dt == 1 && c_dt == 1) hipLaunchKernelGGL((mla_append_kernel<1, 1, NB>), grid, block, 0, s, a);
    else if (in_dt == 1 && c_dt == 2) hipLaunchKernelGGL((mla_append_kernel<1, 2, NB>), grid, block, 0, s, a);
    else if (in_dt == 0 && c_dt == 0) hipLaunchKernelGGL((mla_append_kernel<0, 0, NB>), grid, block, 0, s, a);
    else return -1;
    return 0;
  });
  if (rc != 0) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// The decode kernel instance for (model dtype, cache dtype, rank, fused
// append), as a host function pointer; nullptr for a combination without one.
template <int NB>
const void* decode_kernel(int dt, int c_dt, bool fuse) {
  if (dt == 1 && c_dt == 1 && !fuse)
    return reinterpret_cast<const void*>(&mla_decode_mfma<1, DecodeShape<1, NB>::kDepth, false, NB>);
  if (dt == 1 && c_dt == 2 && !fuse)
    return reinterpret_cast<const void*>(&mla_decode_mfma<2, DecodeShape<2, NB>::kDepth, false, NB>);
  if (dt == 1 && c_dt == 1) return reinterpret_cast<const void*>(&mla_decode_mfma<1, DecodeShape<1, NB>::kDepth, true, NB>);
  if (dt == 1 && c_dt == 2) return reinterpret_cast<const void*>(&mla_decode_mfma<2, DecodeShape<2, NB>::kDepth, true, NB>);
  if (dt == 0 && c_dt == 0 && !fuse) return reinterpret_cast<const void*>(&mla_decode_f32<NB>);
  return nullptr;
}

int launch_decode(const DecodeArgs& a, int dt, int c_dt, hipStream_t s) {
  if (a.n_rows == 0) return 0;
  const dim3 grid = a.balance > 0 ? dim3(a.balance, 1) : dim3(a.n_splits, a.n_rows);
  const bool fuse = a.fa.kv_in != nullptr;
  const int rc = with_nb(a.R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    const void* fn = decode_kernel<NB>(dt, c_dt, fuse);
    if (!fn) return -1;
    void* args[] = {const_cast<DecodeArgs*>(&a)};
    return hipLaunchKernel(fn, grid, dim3(256), args, 0, s) == hipSuccess ? 0 : -2;
  });
  if (rc != 0) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// The workgroups per CU each instance is tuned for (DecodeShape; the fp32
// kernel one), capped by what the device's registers and LDS hold.
int decode_blocks_per_cu(int dt, int c_dt, int R, bool fuse, int* blocks) {
  return with_nb(R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    const void* fn = decode_kernel<NB>(dt, c_dt, fuse);
    if (!fn) return -1;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, 256, 0) != hipSuccess || n < 1) return -2;
    const int tuned = dt == 0 ? 1 : (c_dt == 2 ? DecodeShape<2, NB>::kWavesPerEU : DecodeShape<1, NB>::kWavesPerEU);
    *blocks = n < tuned ? n : tuned;
    return 0;
  });
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
