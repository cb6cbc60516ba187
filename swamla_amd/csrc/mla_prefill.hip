// mla_prefill.hip — gfx950 attention of a prefill chunk over the latent
// cache (reference: models/mla.py:417-487 with seqlen > 1).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "mla_args.h"
#include "mla_device.h"
#include "mla_plan.h"
#include "numerics.h"

namespace swamla {

constexpr int kPrefillQpw = 1;    // queries per wave
constexpr int kPrefillWaves = 8;  // waves (= query groups) per workgroup
constexpr int kPrefillDepth = 1;  // tiles of loads in flight per wave
constexpr int kPrefillOcc = 1;    // workgroups per CU the registers must allow

// ---------------------------------------------------------------------------
// Prefill attention (a chunk of T > 1 new tokens per sequence, dense
// addressing, bf16 model): query token t of sequence b attends causally to
// cache positions [0, start_pos[b] + t + 1) (bottom-right).  A block of NW
// waves takes NW * QPW consecutive query tokens of one sequence, QPW per
// wave, so each 64-token tile of the cache is loaded once for all of them x
// 16 heads.  The tile is staged in LDS (each wave loads
// 64 / NW of its tokens as whole lines); every wave then scores all 64 tokens for its own
// queries (S^T = K . Q^T: each K operand read from LDS feeds QPW MFMAs),
// keeps its own online softmax per (query, head) and accumulates O^T for all
// 256 latent channels (each C^T operand read transposed feeds QPW MFMAs).
// The weights stay in registers: the 8 k slots of lane group g in the PV
// product are tokens 32kb + 4g + {0..3} and 32kb + 16 + 4g + {0..3}, exactly
// the tokens whose scores the lane holds.  No split-KV: the output is o_lat
// directly.  Built with NW = 8 waves of one query each (QPW = 1) and one tile
// of loads in flight: 190 VGPRs, two waves per SIMD; the LDS tiles rotate
// over three buffers so the loop can be software-pipelined (below).
// ---------------------------------------------------------------------------
// One wave's share of a prefill tile: RPL rows of 8 tokens (lane: token l%8,
// 16 bytes at 16(l/8) of each 128-byte segment), plus the rows' e4m3 scales.
// Latent rows of R_pad = 64 NB channels are NB segments (bf16) or ceil(NB / 2)
// (e4m3; for odd NB the last one is half a row).
template <int C_DT, int RPL, int NB>
struct PTile {
  uint4 c[RPL * (C_DT == 2 ? (NB + 1) / 2 : NB)];
  uint4 p[RPL];
  float sc[RPL];
};

template <int C_DT, int DEPTH, int QPW, int NW, int NB>
__global__ __launch_bounds__(NW * 64, kPrefillOcc) void mla_prefill_mfma(DecodeArgs a) {
  constexpr int TPW = kTileTok / NW;  // tokens each wave loads per tile
  constexpr int RPL = TPW / 8;        // ... rows of 8 tokens per lane
  constexpr int SEG = C_DT == 2 ? (NB + 1) / 2 : NB;  // 128-byte latent segments per row
  using Geo = LatGeo<NB, 32>;
  constexpr int RP = Geo::RP, kCRow = Geo::CRow;
  constexpr int CB = C_DT == 2 ? RP : 2 * RP;  // latent bytes per cached token
  constexpr int MB = 4 * NB;                   // 16-channel output blocks
  static_assert(DEPTH == 1, "one tile of loads in flight (the LDS tiles rotate over three buffers)");
  // Three LDS tiles: in iteration j tile j + 1 is stored into one, QK reads
  // it after the iteration's barrier, and PV still reads tile j from another
  // (the third was tile j - 1's, which every wave finished before the
  // barrier).
  constexpr int kBufs = 3;
  __shared__ __attribute__((aligned(16))) uint8_t c_lds2[kBufs][Geo::CBytes];
  __shared__ __attribute__((aligned(16))) uint8_t pe_lds2[kBufs][kPeBytes];
  __shared__ __attribute__((aligned(16))) float sc_lds2[kBufs][kTileTok];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int lt = lane & 7, lc = lane >> 3;
  const int T = a.ad.T;
  const int b = blockIdx.y;
  const int t_first = NW * QPW * blockIdx.x;
  const int t_last_q = min(t_first + NW * QPW - 1, T - 1);  // last query token of the block
  const int sp = a.ad.start_pos[b];
  const bool b_ok = b < a.cache_b;

  // This wave's queries (surplus ones repeat the block's last) and lengths.
  int tq[QPW], rq[QPW], Lq[QPW];
  bool valid[QPW];
#pragma unroll
  for (int qi = 0; qi < QPW; ++qi) {
    const int tt = t_first + QPW * w + qi;
    valid[qi] = tt < T;
    tq[qi] = min(tt, t_last_q);
    rq[qi] = b * T + tq[qi];
    const int l = b_ok ? sp + tq[qi] + 1 : 0;
    Lq[qi] = min(max(l, 0), static_cast<int>(a.cache_s));
  }
  int Lb = b_ok ? sp + t_last_q + 1 : 0;  // the block's range: its last query's
  Lb = min(max(Lb, 0), static_cast<int>(a.cache_s));
  const int n_tiles = (Lb + kTileTok - 1) / kTileTok;  // block-uniform
  const int64_t cache_row0 = static_cast<int64_t>(b_ok ? b : 0) * a.cache_s;
  const int t_last = Lb > 0 ? Lb - 1 : 0;

  auto load_tile = [&](int j, PTile<C_DT, RPL, NB>& kt) {
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) {
      const int64_t row = cache_row0 + min(j * kTileTok + TPW * w + 8 * rr + lt, t_last);
      const uint8_t* cp = static_cast<const uint8_t*>(a.ckv) + row * CB;
#pragma unroll
      for (int q = 0; q < SEG; ++q) {
        const bool half = C_DT == 2 && (NB & 1) && q == SEG - 1;  // upper lanes re-read the first half
        kt.c[rr * SEG + q] = ld_stream16(cp + 128 * q + (half ? 16 * (lc & 3) : 16 * lc));
      }
      kt.p[rr] = ld_stream16(static_cast<const uint8_t*>(a.kpe) + row * (2 * kP) + 16 * lc);
      if constexpr (C_DT == 2) kt.sc[rr] = a.ckv_scale[row];
    }
  };

  // ---- Q^T operands of this wave's queries (lane: head n, 8 channels at 32 kb + 8 g).
  PTile<C_DT, RPL, NB> kt[DEPTH];
  bf16x8_t qb[QPW][2 * NB + 2];
#pragma unroll
  for (int qi = 0; qi < QPW; ++qi) {
    const uint16_t* qa = static_cast<const uint16_t*>(a.q_abs) + rq[qi] * a.qa_rs + n * a.qa_hs;
#pragma unroll
    for (int s = 0; s < 2 * NB; ++s)  // channels >= R zeroed
      qb[qi][s] = as_bf16x8(mask_bf16x8(*reinterpret_cast<const uint4*>(qa + 32 * s + 8 * g), a.R - (32 * s + 8 * g)));
  }
  uint4 raw[QPW][2];
  uint2 cr[QPW][2], sr[QPW][2];
#pragma unroll
  for (int qi = 0; qi < QPW; ++qi) {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q_pe) + rq[qi] * a.qp_rs + n * a.qp_hs;
    int rp = a.ad.rope_abs ? sp + tq[qi] : tq[qi];
    rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
    const uint16_t* ct = static_cast<const uint16_t*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
    const uint16_t* st = static_cast<const uint16_t*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c0 = 32 * s + 8 * g;
      raw[qi][s] = *reinterpret_cast<const uint4*>(qp + c0);
      cr[qi][s] = *reinterpret_cast<const uint2*>(ct + c0 / 2);
      sr[qi][s] = *reinterpret_cast<const uint2*>(st + c0 / 2);
    }
  }
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_tile(d, kt[d]);
#pragma unroll
  for (int qi = 0; qi < QPW; ++qi)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t wv_in[4] = {raw[qi][s].x, raw[qi][s].y, raw[qi][s].z, raw[qi][s].w};
      const uint32_t cw2[2] = {cr[qi][s].x, cr[qi][s].y}, sw2[2] = {sr[qi][s].x, sr[qi][s].y};
      uint32_t wv[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint32_t cj = (jj & 1) ? (cw2[jj >> 1] >> 16) : (cw2[jj >> 1] & 0xFFFF);
        const uint32_t sj = (jj & 1) ? (sw2[jj >> 1] >> 16) : (sw2[jj >> 1] & 0xFFFF);
        wv[jj] = rope_bf16_packed(bf16_to_f32(wv_in[jj] & 0xFFFF), bf16_to_f32(wv_in[jj] >> 16), bf16_to_f32(cj),
                                  bf16_to_f32(sj));
      }
      qb[qi][2 * NB + s] = as_bf16x8(make_uint4(wv[0], wv[1], wv[2], wv[3]));
    }

  f32x4_t oacc[QPW][MB];
#pragma unroll
  for (int qi = 0; qi < QPW; ++qi)
#pragma unroll
    for (int i = 0; i < MB; ++i) oacc[qi][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[QPW], l_part[QPW];
#pragma unroll
  for (int qi = 0; qi < QPW; ++qi) {
    m_run[qi] = -INFINITY;
    l_part[qi] = 0.f;
  }

  // This wave's rows of a loaded tile (e4m3 decoded to bf16, with their
  // scales) into LDS buffer bf.
  auto store_tile = [&](int bf, const PTile<C_DT, RPL, NB>& kt) {
    uint8_t* const c_st = c_lds2[bf] + (TPW * w + lt) * kCRow + 16 * lc;
    uint8_t* const pe_st = pe_lds2[bf] + (TPW * w + lt) * kPeRow + 16 * lc;
    float* const sc_lds = sc_lds2[bf];
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) {
      if constexpr (C_DT == 2) {
#pragma unroll
        for (int q = 0; q < SEG; ++q) {
          const uint4 v = kt.c[rr * SEG + q];
          const uint2 a0 = e4m3x4_to_bf16x4_hw(v.x), a1 = e4m3x4_to_bf16x4_hw(v.y);
          const uint2 a2 = e4m3x4_to_bf16x4_hw(v.z), a3 = e4m3x4_to_bf16x4_hw(v.w);
          if ((NB & 1) && q == SEG - 1 && lc >= 4) continue;  // the re-read half is not stored
          uint8_t* dst = c_st + 8 * rr * kCRow + 2 * (128 * q);  // channels 128q + 16lc .. +16
          *reinterpret_cast<uint4*>(dst + 16 * lc) = make_uint4(a0.x, a0.y, a1.x, a1.y);
          *reinterpret_cast<uint4*>(dst + 16 * lc + 16) = make_uint4(a2.x, a2.y, a3.x, a3.y);
        }
        if (lc == 0) sc_lds[TPW * w + 8 * rr + lt] = kt.sc[rr];
      } else {
#pragma unroll
        for (int q = 0; q < SEG; ++q) {
          const uint4 v = kt.c[rr * SEG + q];
          *reinterpret_cast<uint4*>(c_st + 8 * rr * kCRow + 128 * q) = make_uint4(v.x, v.y, v.z, v.w);
        }
      }
      const uint4 pv = kt.p[rr];
      *reinterpret_cast<uint4*>(pe_st + 8 * rr * kPeRow) = make_uint4(pv.x, pv.y, pv.z, pv.w);
    }
  };

  // Tile j lives in LDS buffer j % 3.
  // qk(j, x): scores of all 64 tokens of tile j for this wave's queries
  // (token 16tb + 4g + i, head n), masked and scaled to the log2 domain.
  float x[QPW][4][4];
  bf16x8_t pb[QPW][2];
  auto qk = [&](int j) {
    const int bf = j % kBufs;
    const uint8_t* const c_lds = c_lds2[bf];
    const uint8_t* const pe_lds = pe_lds2[bf];
    const float* const sc_lds = sc_lds2[bf];
    // operand reads of token block tb: token 16tb + n, 8 channels at 32s + 8g
    const uint8_t* const c_op = c_lds + n * kCRow + 2 * (8 * g);
    const uint8_t* const pe_op = pe_lds + n * kPeRow + 2 * (8 * g);
    const int tile0 = j * kTileTok;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      f32x4_t s_c[QPW], s_p[QPW];
#pragma unroll
      for (int qi = 0; qi < QPW; ++qi) s_c[qi] = s_p[qi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2 * NB; ++s) {
        const bf16x8_t ka = as_bf16x8(*reinterpret_cast<const uint4*>(c_op + 16 * tb * kCRow + 2 * (32 * s)));
#pragma unroll
        for (int qi = 0; qi < QPW; ++qi) s_c[qi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[qi][s], s_c[qi], 0, 0, 0);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8_t pa = as_bf16x8(*reinterpret_cast<const uint4*>(pe_op + 16 * tb * kPeRow + 2 * (32 * s)));
#pragma unroll
        for (int qi = 0; qi < QPW; ++qi)
          s_p[qi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, qb[qi][2 * NB + s], s_p[qi], 0, 0, 0);
      }
      float4 scv = make_float4(1.f, 1.f, 1.f, 1.f);
      if constexpr (C_DT == 2) scv = *reinterpret_cast<const float4*>(sc_lds + 16 * tb + 4 * g);
      const float sc4[4] = {scv.x, scv.y, scv.z, scv.w};
#pragma unroll
      for (int qi = 0; qi < QPW; ++qi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sv = (C_DT == 2) ? (sc4[i] * s_c[qi][i] + s_p[qi][i]) : (s_c[qi][i] + s_p[qi][i]);
          const int tok = tile0 + 16 * tb + 4 * g + i;
          x[qi][tb][i] = tok < Lq[qi] ? sv * a.scale_log2 : -INFINITY;
        }
    }
  };
  // softmax(j): the online-softmax step of tile j's scores x: running max
  // (rescaling O when it moves), weight sums, and the bf16 weights pb in the
  // PV operand order.
  auto softmax = [&](int j) {
    const float* const sc_lds = sc_lds2[j % kBufs];
    (void)sc_lds;
#pragma unroll
    for (int qi = 0; qi < QPW; ++qi) {
      float mt = -INFINITY;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mt = fmaxf(mt, x[qi][tb][i]);
      mt = wave_max_rows(mt);  // this query's tile maximum for head n
      if (__any(mt > m_run[qi] + kLazy)) {
        const float m_new = fmaxf(m_run[qi], mt);
        const float alpha = exp2f(m_run[qi] - m_new);  // m_new is finite: mt is
        m_run[qi] = m_new;
        l_part[qi] *= alpha;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) oacc[qi][mb] = oacc[qi][mb] * alpha;
      }
      // bf16 weights (fp8: times the token's scale) in the PV operand order.
      // A query with no valid token yet (m_run still -inf: only a negative
      // start position gives one) takes weight 0 for every token, not NaN.
      const float mref = m_run[qi] == -INFINITY ? 0.f : m_run[qi];
      uint2 pw[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = exp2f(x[qi][tb][i] - mref);
        const uint32_t w01 = pack_bf16x2(pr[0], pr[1]), w23 = pack_bf16x2(pr[2], pr[3]);
        l_part[qi] += (u2f(w01 << 16) + u2f(w01 & 0xFFFF0000u)) + (u2f(w23 << 16) + u2f(w23 & 0xFFFF0000u));
        if constexpr (C_DT == 2) {
          const float4 scv = *reinterpret_cast<const float4*>(sc_lds + 16 * tb + 4 * g);
          pw[tb].x = pack_bf16x2(u2f(w01 << 16) * scv.x, u2f(w01 & 0xFFFF0000u) * scv.y);
          pw[tb].y = pack_bf16x2(u2f(w23 << 16) * scv.z, u2f(w23 & 0xFFFF0000u) * scv.w);
        } else {
          pw[tb] = make_uint2(w01, w23);
        }
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        pb[qi][kb] = as_bf16x8(make_uint4(pw[2 * kb].x, pw[2 * kb].y, pw[2 * kb + 1].x, pw[2 * kb + 1].y));
    }
  };
  // pv(j): O^T[16mb + ., head] += C^T . P^T over tile j's two 32-token halves.
  auto pv = [&](int j) {
    // C^T reads: token row 4g + n/4 of each 16-token block, channel 4(n%4) (+16 mb)
    const uint8_t* const c_tr = c_lds2[j % kBufs] + (4 * g + (n >> 2)) * kCRow + 8 * (n & 3);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const s16x4_t c0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4_t*)(c_tr + (32 * kb) * kCRow + 32 * mb));
        const s16x4_t c1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4_t*)(c_tr + (32 * kb + 16) * kCRow + 32 * mb));
        const bf16x8_t cv = cat_bf16x8(c0, c1);
#pragma unroll
        for (int qi = 0; qi < QPW; ++qi)
          oacc[qi][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cv, pb[qi][kb], oacc[qi][mb], 0, 0, 0);
      }
    }
  };

  // Software-pipelined over tiles: the prologue stores tile 0, issues tile
  // 1's loads and runs tile 0's scores and softmax.  Iteration j stores tile
  // j + 1 (loaded during iteration j - 1) into its buffer and issues tile
  // j + 2's loads; after the barrier (tile j + 1 visible, tile j - 1's buffer
  // free) the wave issues tile j + 1's QK MFMAs and tile j's PV MFMAs back to
  // back, then tile j + 1's softmax, whose VALU work overlaps the PV MFMAs
  // still in flight.  Loads past the last tile re-read its last rows (in
  // bounds, never stored).
  if (n_tiles > 0) {
    store_tile(0, kt[0]);
    load_tile(1, kt[0]);
    lds_barrier();
    qk(0);
    softmax(0);
  }
  for (int j = 0; j < n_tiles; ++j) {  // block-uniform
    const bool more = j + 1 < n_tiles;
    if (more) {
      store_tile((j + 1) % kBufs, kt[0]);
      load_tile(j + 2, kt[0]);
    }
    lds_barrier();
    if (more) qk(j + 1);
    pv(j);
    if (more) softmax(j + 1);
  }

#pragma unroll
  for (int qi = 0; qi < QPW; ++qi) {
    float l_w = l_part[qi] + shfl_xor_f32(l_part[qi], 16);
    l_w += shfl_xor_f32(l_w, 32);
    const float inv = l_w > 0.f ? 1.f / l_w : 0.f;
    if (valid[qi]) {
      // lane (n, g): head n, channels 16mb + 4g + {0..3}
      uint16_t* op = static_cast<uint16_t*>(a.o_lat) + rq[qi] * a.o_rs + n * a.o_hs + 4 * g;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        uint2 pk;
        pk.x = f32_to_bf16(oacc[qi][mb][0] * inv) | (static_cast<uint32_t>(f32_to_bf16(oacc[qi][mb][1] * inv)) << 16);
        pk.y = f32_to_bf16(oacc[qi][mb][2] * inv) | (static_cast<uint32_t>(f32_to_bf16(oacc[qi][mb][3] * inv)) << 16);
        *reinterpret_cast<uint2*>(op + 16 * mb) = pk;
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Prefill attention on 32x32x16 MFMAs (bf16 cache, R_pad a multiple of 128).
// A workgroup of four waves (one per SIMD) takes eight consecutive query
// tokens of one sequence, two per wave: the wave's 32 MFMA columns are
// (query, head) = (n >> 4, n & 15).  Per 64-token cache tile, staged in LDS
// once for the workgroup (each wave loads 16 of the rows as whole lines):
//   S^T[32 tok x 32 col] = K . Q^T   two 32-token halves, A = K rows from
//                                    LDS, B = Q^T in registers for the whole
//                                    walk (R_pad / 16 + 4 k-steps);
//   online softmax per column        the lane holds 16 tokens of its column
//                                    per half-tile, the other lane half the
//                                    other 16 (one permlane32 swap);
//   O^T[32 ch x 32 col] += V^T . P^T per 32-channel block, A = C^T read
//                                    transposed from LDS (ds_read_b64_tr_b16),
//                                    B = the bf16 weights straight from the
//                                    score registers.
// The score accumulator's lane layout (row 8(r/4) + 4(l/32) + r%4, column
// l%32) is the PV product's B operand once the k slots of the 16-token step
// are taken as tokens {4h .. 4h+3, 8+4h .. 8+4h+3} for lane half h, which is
// also the order in which the two transposed reads of C^T deliver them.  Each
// K or C^T byte read from LDS feeds 32 columns instead of 16, so the tile's
// LDS traffic per query is half that of mla_prefill_mfma.
// LDS: latent rows at a 2 R_pad pitch with 16-byte chunk c of row t at
// (c & ~15) | ((c ^ p2_swz(t)) & 15): the K read (one chunk of 16 rows per
// 16 lanes) and the transposed read (4 rows x 64 bytes per 32 lanes) both
// hit 64 distinct banks (measured: no bank conflicts); rope rows (128 bytes)
// at chunk c ^ ((t >> 1) & 7).  The rows arrive by LDS DMA
// (global_load_lds_dwordx4, 1 KB per instruction, the swizzle applied to the
// global addresses), so no register or LDS-store instruction stages them.
// Three tile buffers: iteration j waits for its own DMAs of tile j + 1,
// passes one barrier, starts tile j + 2's DMAs into the buffer tile j - 1
// left, then runs tile j + 1's QK and tile j's PV back to back.  The operand
// reads run a fixed number of MFMAs ahead with explicit waits, and the
// softmax step of tile j + 1 is placed between PV MFMAs, where its VALU work
// overlaps the matrix pipe.  Each wave is alone on its SIMD (about 230
// VGPRs and 240 AGPRs: O^T, the scores and Q^T live in AGPRs, from which the
// MFMAs read directly).
// ---------------------------------------------------------------------------
namespace {
typedef float f32x16_t __attribute__((ext_vector_type(16)));
constexpr int kP2Waves = 4;  // waves per workgroup, one per SIMD
constexpr int kP2Qpw = 2;    // query tokens per wave (x 16 heads = 32 MFMA columns)
constexpr int kP2Tok = 64;   // cache tokens per LDS tile
constexpr int kP2Bufs = 3;

__device__ __forceinline__ int p2_swz(int t) { return ((t & 3) << 2) | ((t >> 2) & 3); }
typedef unsigned int p2_u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
// LDS operand reads issued as inline assembly, so that their order and the
// waits for them are the source's: the compiler would otherwise keep one
// read in flight per MFMA.  Results are taken only after p2_wait_lgkm<N>()
// (LDS operations complete in order) and p2_tie(), which redefines the value
// so that no use moves above the wait.
template <int OFF>
__device__ __forceinline__ p2_u32x4_t p2_read16(uint32_t addr) {
  p2_u32x4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <int OFF>
__device__ __forceinline__ s16x4_t p2_read_tr(uint32_t addr) {
  s16x4_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void p2_wait_lgkm() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}
template <typename T>
__device__ __forceinline__ void p2_tie(T& v) { asm volatile("" : "+v"(v)); }
// s_waitcnt vmcnt(N) alone (gfx9 encoding)
template <int N>
__device__ __forceinline__ void p2_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// 8-byte store as inline assembly (one vector-memory instruction whatever
// the compiler would make of it: the prologue's vmcnt waits count them)
template <int OFF>
__device__ __forceinline__ void p2_store8(void* p, uint32_t lo, uint32_t hi) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  const u32x2_t v = {lo, hi};
  asm volatile("global_store_dwordx2 %0, %1, off offset:%2" ::"v"(p), "v"(v), "i"(OFF) : "memory");
}
// 16 bytes per lane from global memory into LDS at dst + 16 lane (cacheable:
// the workgroups of one sequence read the same rows)
__device__ __forceinline__ void p2_dma16(const void* src, lds_u8* dst) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<lds_void*>(dst), 16, 0, 0);
}
template <int I, int N, typename F>
__device__ __forceinline__ void p2_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    p2_for<I + 1, N>(f);
  }
}
template <int A, int B>
constexpr int p2_min() { return A < B ? A : B; }
// LDS reads issued for stream slots 0 .. i when the first QK slots take one
// read each and the rest two
template <int QK>
constexpr int p2_nreads(int i) { return i < QK ? i + 1 : QK + 2 * (i - QK + 1); }
__device__ __forceinline__ int p2_pos(int c, int t) { return (c & ~15) | ((c ^ p2_swz(t)) & 15); }
}  // namespace

template <int NB>
__global__ __launch_bounds__(kP2Waves * 64, 1) void mla_prefill_m32(DecodeArgs a) {
  static_assert(NB % 2 == 0, "latent rows of a multiple of 256 bytes");
  constexpr int RP = 64 * NB;
  constexpr int kRow = 2 * RP;                  // bytes per latent row
  constexpr int kLat = kP2Tok * kRow;           // latent bytes per tile
  constexpr int kPeR = 2 * kP;                  // bytes per rope row
  constexpr int kBuf = kLat + kP2Tok * kPeR;    // bytes per tile buffer
  constexpr int KS = RP / 16;                   // latent k-steps of the QK product
  constexpr int CB = RP / 32;                   // 32-channel blocks of the PV product
  constexpr int LQ = 16 * kRow / 1024;          // latent DMAs per wave per tile (16 rows)
  constexpr int kRowsPerDma = 1024 / kRow;
  constexpr int QG = kP2Waves * kP2Qpw;         // query tokens per workgroup
  // Three buffers as three arrays: every access names its array at compile
  // time (the loop is unrolled by three), so the compiler's wait counting can
  // tell a read of one buffer from the DMA still filling another.
  __shared__ __attribute__((aligned(16))) uint8_t lds0[kBuf];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[kBuf];
  __shared__ __attribute__((aligned(16))) uint8_t lds2[kBuf];
  // the query rows' staging area of waves 2 and 3 (waves 0 and 1 stage theirs
  // in lds2, whose first tile arrives after the loop's first barrier)
  __shared__ __attribute__((aligned(16))) uint8_t lds3[kBuf];
  auto buf = [&](auto bi) __attribute__((always_inline)) -> lds_u8* {
    if constexpr (decltype(bi)::value == 0) return (lds_u8*)lds0;
    else if constexpr (decltype(bi)::value == 1) return (lds_u8*)lds1;
    else return (lds_u8*)lds2;
  };

  const int T = a.ad.T;
  // Persistent workgroups: item k is query group G - 1 - k / B of row k % B
  // (the later query groups, which attend to more of the cache, come
  // first), and workgroup x takes items r X + x in even rounds r and
  // r X + X - 1 - x in odd ones (X workgroups), so each pair of rounds deals
  // every workgroup about the same number of tiles.
  const int n_groups = (T + QG - 1) / QG;
  const int B = a.n_rows / T;
  const int n_items = n_groups * B;
  // An item's output stores are issued at the next item's start, after its
  // loads (the vmcnt waits for those loads then do not wait for the stores).
  constexpr int kStores = CB * 4;  // 8-byte stores per lane and item
  bool pending = false;            // uniform
  uint32_t pend[CB][4][2];
  uint16_t* pend_op = nullptr;
  auto flush = [&]() __attribute__((always_inline)) {
    p2_for<0, CB>([&](auto cbI) {
      constexpr int cb = decltype(cbI)::value;
      p2_for<0, 4>([&](auto r4I) {
        constexpr int r4 = decltype(r4I)::value;
        p2_store8<2 * (32 * cb + 8 * r4)>(pend_op, pend[cb][r4][0], pend[cb][r4][1]);
      });
    });
  };
  for (int round = 0;; ++round) {
    const int item = round * static_cast<int>(gridDim.x) +
                     ((round & 1) ? static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x)
                                  : static_cast<int>(blockIdx.x));
    if (item >= n_items) break;  // uniform
    // The lane's indices are re-derived per item from an opaque copy of the
    // thread id: nothing computed from them is hoisted out of the item loop
    // and kept live across it (the body uses every register).
    int tid = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid));
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int n = lane & 31, hf = lane >> 5;  // column, lane half
    const int head = n & 15;
    const int b = item % B;
    const int t_first = QG * (n_groups - 1 - item / B);
    const int t_last_q = min(t_first + QG - 1, T - 1);
    const int sp = a.ad.start_pos[b];
    const bool b_ok = b < a.cache_b;
    const int tt = t_first + kP2Qpw * w + (n >> 4);  // this column's query (surplus ones repeat the last)
    const int tq = min(tt, t_last_q);
    const int64_t rq = static_cast<int64_t>(b) * T + tq;
    int Lq = b_ok ? sp + tq + 1 : 0;
    Lq = min(max(Lq, 0), static_cast<int>(a.cache_s));
    int Lb = b_ok ? sp + t_last_q + 1 : 0;  // the block's range: its last query's
    Lb = min(max(Lb, 0), static_cast<int>(a.cache_s));
    const int n_tiles = (Lb + kP2Tok - 1) / kP2Tok;  // block-uniform
    const int64_t cache_row0 = static_cast<int64_t>(b_ok ? b : 0) * a.cache_s;
    const int t_last = Lb > 0 ? Lb - 1 : 0;
    // this sequence's cache rows (32-bit lane offsets from a uniform base)
    const uint8_t* const ckv = static_cast<const uint8_t*>(a.ckv) + cache_row0 * kRow;
    const uint8_t* const kpe = static_cast<const uint8_t*>(a.kpe) + cache_row0 * kPeR;

    // ---- DMA of this wave's 16 rows of tile j (rows 16w .. 16w + 15) straight
    // into LDS, 1 KB per instruction: LDS chunk p of row t holds cache chunk
    // p ^ swizzle(t) (the XOR is its own inverse).
    uint32_t lat_src[LQ], pe_src[2];  // lane offsets within a tile's rows, row index excluded
    int lat_row[LQ], pe_row[2];
#pragma unroll
    for (int q = 0; q < LQ; ++q) {
      const int t = 16 * w + kRowsPerDma * q + (16 * lane) / kRow, pch = ((16 * lane) % kRow) / 16;
      lat_row[q] = t;
      lat_src[q] = 16 * p2_pos(pch, t);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int t = 16 * w + 8 * q + (lane >> 3);
      pe_row[q] = t;
      pe_src[q] = 16 * ((lane & 7) ^ ((t >> 1) & 7));
    }
    auto dma_tile = [&](int j, lds_u8* dst) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < LQ; ++q) {
        const uint32_t row = min(j * kP2Tok + lat_row[q], t_last);
        p2_dma16(ckv + (row * kRow + lat_src[q]), dst + (16 * w + kRowsPerDma * q) * kRow);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t row = min(j * kP2Tok + pe_row[q], t_last);
        p2_dma16(kpe + (row * kPeR + pe_src[q]), dst + kLat + (16 * w + 8 * q) * kPeR);
      }
    };

    // ---- Q^T operands: column n (query n >> 4 of the wave, head n & 15),
    // channels 16 ks + 8 hf .. + 7 (k-steps KS.. are the rope part).  The
    // wave's 32 query rows are copied into its staging area by LDS DMA in whole
    // lines (1 KB per instruction): column n's latent chunk c at slot (c & 16) |
    // ((c ^ n) & 15), its rope chunk c at (c ^ (n >> 1)) & 7, so that the
    // operand reads (chunk 2 ks + hf of 16 columns per read cycle) hit distinct
    // banks.  Loaded per lane instead, 16 bytes of 32 rows per instruction, the
    // rows took several microseconds per item.
    constexpr int kQLat = 32 * kRow;                // latent bytes of the wave's 32 columns
    constexpr int kQBytes = kQLat + 32 * kPeR;
    constexpr int kQDma = kQBytes / 1024;           // DMA instructions for the wave's rows
    static_assert(kQLat % 1024 == 0 && 2 * kQBytes <= kBuf, "two waves' rows fit a staging buffer");
    lds_u8* const qs = ((w >> 1) == 0 ? (lds_u8*)lds2 : (lds_u8*)lds3) + (w & 1) * kQBytes;
    const int tq_w = min(t_first + kP2Qpw * w, t_last_q);  // the wave's first query (surplus ones repeat the last)
    const int64_t rq_w = static_cast<int64_t>(b) * T + tq_w;
    const int rq_step = min(t_first + kP2Qpw * w + 1, t_last_q) - tq_w;  // 0 or 1
    p2_for<0, kQDma>([&](auto iI) {
      constexpr int i = decltype(iI)::value;
      const int o = 1024 * i + 16 * lane;
      if constexpr (1024 * i < kQLat) {
        const int col = o / kRow, sl = (o % kRow) / 16, ch = (sl & 16) | ((sl ^ col) & 15);
        const uint16_t* src = static_cast<const uint16_t*>(a.q_abs) + (rq_w + (col >> 4) * rq_step) * a.qa_rs +
                              (col & 15) * a.qa_hs + 8 * ch;
        p2_dma16(src, qs + 1024 * i);
      } else {
        const int o2 = o - kQLat, col = o2 / kPeR, ch = ((o2 % kPeR) / 16 ^ (col >> 1)) & 7;
        const uint16_t* src = static_cast<const uint16_t*>(a.q_pe) + (rq_w + (col >> 4) * rq_step) * a.qp_rs +
                              (col & 15) * a.qp_hs + 8 * ch;
        p2_dma16(src, qs + 1024 * i);
      }
    });
    // the RoPE row of the column's query (cos / sin as 4 x 2 words each)
    uint32_t cr[4][2], sr[4][2];
    {
      int rp = a.ad.rope_abs ? sp + tq : tq;
      rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
      const uint16_t* ct = static_cast<const uint16_t*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
      const uint16_t* st = static_cast<const uint16_t*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        vm_load<2>(ct + (16 * s4 + 8 * hf) / 2, cr[s4]);
        vm_load<2>(st + (16 * s4 + 8 * hf) / 2, sr[s4]);
      }
    }
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    // tiles 0 and 1 (a tile past the last, or with no tile at all, re-reads an
    // in-bounds row), then the previous item's output
    dma_tile(0, buf(I0{}));
    dma_tile(1, buf(I1{}));
    // in flight, in issue order: query rows (kQDma), cos / sin (8), tile 0 and
    // tile 1 (LQ + 2 each); then the previous item's stores (kStores), issued
    // once the query rows are in (queued ahead of them, the stores held back
    // their arrival)
    constexpr int kTileVm = LQ + 2;
    p2_wait_vm<8 + 2 * kTileVm>();
    const bool flushed = pending;  // uniform
    if (flushed) flush();
    bf16x8_t qb[KS + 4];
    {
      const uint32_t q0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(qs)) + n * kRow;
      const int nx = (n ^ hf) & 15;  // (2 ks + hf) ^ n = 2 ks ^ (n ^ hf) on the low four bits
      p2_u32x4_t qr[KS + 4];
      p2_for<0, KS>([&](auto ksI) {
        constexpr int ks = decltype(ksI)::value;
        qr[ks] = p2_read16<16 * ((2 * ks) & 16)>(q0 + 16 * (((2 * ks) & 15) ^ nx));
      });
      const uint32_t p0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(qs)) + kQLat + n * kPeR;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) qr[KS + s4] = p2_read16<0>(p0 + 16 * (((2 * s4 + hf) ^ (n >> 1)) & 7));
      p2_wait_lgkm<0>();
#pragma unroll
      for (int ks = 0; ks < KS + 4; ++ks) p2_tie(qr[ks]);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)  // channels >= R zeroed
        qb[ks] = as_bf16x8(mask_bf16x8(make_uint4(qr[ks].x, qr[ks].y, qr[ks].z, qr[ks].w), a.R - (16 * ks + 8 * hf)));
      if (flushed) p2_wait_vm<2 * kTileVm + kStores>();
      else p2_wait_vm<2 * kTileVm>();
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        vm_release(cr[s4]);
        vm_release(sr[s4]);
        const uint32_t wv_in[4] = {qr[KS + s4].x, qr[KS + s4].y, qr[KS + s4].z, qr[KS + s4].w};
        uint32_t wv[4];
#pragma unroll
        for (int j2 = 0; j2 < 4; ++j2) {
          const uint32_t cj = (j2 & 1) ? (cr[s4][j2 >> 1] >> 16) : (cr[s4][j2 >> 1] & 0xFFFF);
          const uint32_t sj = (j2 & 1) ? (sr[s4][j2 >> 1] >> 16) : (sr[s4][j2 >> 1] & 0xFFFF);
          wv[j2] = rope_bf16_packed(bf16_to_f32(wv_in[j2] & 0xFFFF), bf16_to_f32(wv_in[j2] >> 16), bf16_to_f32(cj),
                                    bf16_to_f32(sj));
        }
        qb[KS + s4] = as_bf16x8(make_uint4(wv[0], wv[1], wv[2], wv[3]));
      }
#pragma unroll
      for (int ks = 0; ks < KS + 4; ++ks) asm volatile("" : "+a"(qb[ks]));  // kept in AGPRs: MFMA reads B from there
    }
    pending = false;

    f32x16_t oacc[CB];
#pragma unroll
    for (int i = 0; i < CB; ++i) oacc[i] = f32x16_t{};
    float m_run = -INFINITY, l_part = 0.f;

    // ---- per-lane operand offsets (bytes within a tile buffer).  The swizzle
    // XORs only the low four bits of a chunk index, so each read is a per-lane
    // table entry plus a compile-time offset (the ds_read immediate):
    //   K latent, k-step ks, half h2: ko[ks % 8] + 256 (ks / 8) + 32 h2 kRow
    //   K rope, k-step s, half h2:    po[s] + 32 h2 kPeR
    //   C^T, k-step s, block cb, read e: to[e][cb % 4] + 16 s kRow + 256 (cb / 4)
    const int fl = p2_swz(n & 15);  // rows 32 h2 + n of a tile
    const int pe_sw = (n >> 1) & 7;
    const int G = lane >> 4, jj = lane & 15, g2 = G & 1;  // transposed reads: 16-lane group, lane in group
    uint32_t ko[8], po[4], to[2][4];
#pragma unroll
    for (int k8 = 0; k8 < 8; ++k8) ko[k8] = n * kRow + 16 * ((2 * k8 + hf) ^ fl);
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) po[s4] = kLat + n * kPeR + 16 * ((2 * s4 + hf) ^ pe_sw);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 8 * e + 4 * hf + (jj >> 2);  // row within a 16-token k-step
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4)
        to[e][c4] = r * kRow + 16 * ((4 * c4 + 2 * g2 + ((jj & 3) >> 1)) ^ p2_swz(r)) + 8 * (jj & 1);
    }
    static_assert(KS <= 16 && kRow % 256 == 0, "the latent read table covers 16 k-steps of 256-byte row halves");

    // qk(j, base): scores of tile j, scaled to the log2 domain and masked.
    // The 2 (KS + 4) K reads run kQkAhead ahead of their MFMAs.
    constexpr int kQkReads = 2 * (KS + 4), kQkAhead = 6;
    f32x16_t sc[2];
    int sc_tile = 0;  // the tile sc holds (scaled and masked in the softmax step)
    auto qk = [&](int j, const lds_u8* base_p) __attribute__((always_inline)) {
      const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(base_p));
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) sc[h2] = f32x16_t{};
      p2_u32x4_t kr[kQkReads];
      auto rd = [&](auto I) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value, ks = i / 2, h2 = i % 2;
        if constexpr (ks < KS) kr[i] = p2_read16<256 * (ks / 8) + 32 * h2 * kRow>(base + ko[ks % 8]);
        else kr[i] = p2_read16<32 * h2 * kPeR>(base + po[ks - KS]);
      };
      p2_for<0, kQkAhead>(rd);
      p2_for<0, kQkReads>([&](auto I) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value, ks = i / 2, h2 = i % 2;
        if constexpr (i + kQkAhead < kQkReads) {
          rd(std::integral_constant<int, i + kQkAhead>{});
          p2_wait_lgkm<kQkAhead>();
        } else {
          p2_wait_lgkm<kQkReads - 1 - i>();
        }
        p2_tie(kr[i]);
        sc[h2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kr[i]), qb[ks], sc[h2], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      });
      sc_tile = j;
    };
    // smax(): the online-softmax step of the scores sc, without touching O:
    // the new reference m_new (moved lazily, when a column's maximum grows by
    // more than 2^kLazy), the rescale factor alpha of what was accumulated so
    // far, and the bf16 weights pbn in the PV operand order (k-step s = 2 h2 +
    // sb: registers 8 sb .. 8 sb + 7 of half h2) with their sum.  The caller
    // rescales O after the PV product of the previous tile, which used the old
    // reference.  Branch-free, so it shares one scheduling region with that
    // product.
    bf16x8_t pb[4], pbn[4];
    float alpha = 1.f, lsum = 0.f, m_new = -INFINITY;
    bool moved = false;
    // part 0: the tile maximum and the new reference; parts 1, 2: the weights
    // of half-tile 0, 1
    float mref = 0.f;
    auto smax_part = [&](auto P) __attribute__((always_inline)) {
      constexpr int part = decltype(P)::value;
      if constexpr (part == 0) {
        // Tokens at or past a column's causal end score -inf; only the tiles
        // that reach the end of one of the wave's queries need the compares.
        if (!__all(sc_tile * kP2Tok + kP2Tok <= Lq)) {
          const int tok0 = sc_tile * kP2Tok + 4 * hf;
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int tok = tok0 + 32 * h2 + 8 * (r >> 2) + (r & 3);
              if (tok >= Lq) sc[h2][r] = -INFINITY;
            }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[h2][r]);
        const uint32_t u = f2u(mt);
        const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        // the column's tile maximum (both lane halves), in the log2 domain (the scale is positive)
        mt = fmaxf(u2f(r32[0]), u2f(r32[1])) * a.scale_log2;
        // Each column moves its own reference, only when its maximum grew by
        // more than kLazy: its arithmetic then depends on its own scores
        // alone, so a surplus column (repeating the block's last query, in
        // this wave or another) computes that query's output bit for bit.
        const bool mine = mt > m_run + kLazy;
        moved = __any(mine);
        m_new = mine ? fmaxf(m_run, mt) : m_run;
        // a column that keeps its reference (or is still without a valid
        // token: both -inf) keeps alpha = 1, not NaN
        alpha = m_new == m_run ? 1.f : exp2f(m_run - m_new);
        // A column with no valid token yet (reference still -inf) takes weight 0, not NaN.
        mref = m_new == -INFINITY ? 0.f : -m_new;  // (negated: the weights are exp2(s scale - m))
        lsum = 0.f;
        p2_tie(mref);  // keeps this part where it is placed (the compiler would sink it to its uses)
        p2_tie(alpha);
      } else {
        constexpr int h2 = part - 1;
        // weights exp2(s scale - m) with one rounding before the exponential
        // (v_exp_f32: the arguments are at most kLazy, so no range reduction),
        // rounded to bf16; their sum with one dot2 per pair
        const bf16x2_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          uint32_t pw[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[h2][8 * sb + 2 * e], a.scale_log2, mref));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[h2][8 * sb + 2 * e + 1], a.scale_log2, mref));
            pw[e] = pack_bf16x2(p0, p1);
            lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pw[e]), ones, lsum, false);
          }
          pbn[2 * h2 + sb] = as_bf16x8(make_uint4(pw[0], pw[1], pw[2], pw[3]));
          p2_tie(pbn[2 * h2 + sb]);
        }
        p2_tie(lsum);
      }
    };
    auto smax = [&]() __attribute__((always_inline)) {
      smax_part(std::integral_constant<int, 0>{});
      smax_part(std::integral_constant<int, 1>{});
      smax_part(std::integral_constant<int, 2>{});
    };
    // the softmax parts placed after PV MFMAs M/8, 3M/8 and 5M/8 (M = 4 CB)
    auto smax_mid = [&](auto I) __attribute__((always_inline)) {
      constexpr int m = decltype(I)::value, M = 4 * CB;
      if constexpr (m == M / 8) smax_part(std::integral_constant<int, 0>{});
      else if constexpr (m == 3 * M / 8) smax_part(std::integral_constant<int, 1>{});
      else if constexpr (m == 5 * M / 8) smax_part(std::integral_constant<int, 2>{});
    };
    // commit(): the reference and weight sum move to the new tile; O is
    // rescaled if any column's reference moved (rare after the first tiles;
    // the other columns' alpha is 1).
    auto commit = [&]() __attribute__((always_inline)) {
      l_part = l_part * alpha + lsum;
      m_run = m_new;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) pb[s4] = pbn[s4];
      if (moved) {
#pragma unroll
        for (int i = 0; i < CB; ++i) {  // one block at a time: few registers live
          oacc[i] = oacc[i] * alpha;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    // pv(base, mid): O^T[32 cb + ., col] += C^T . P^T over a tile's four
    // 16-token k-steps, the two transposed reads of each MFMA kPvAhead MFMAs
    // ahead; mid(I) runs after MFMA I (the next tile's softmax work, which
    // then overlaps the MFMAs in flight).
    constexpr int kPvMfma = 4 * CB, kPvAhead = 6;
    auto pv = [&](const lds_u8* base_p, auto&& mid) __attribute__((always_inline)) {
      const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(base_p));
      s16x4_t cr[kPvMfma][2];
      auto rd = [&](auto I) __attribute__((always_inline)) {
        constexpr int m = decltype(I)::value, s4 = m / CB, cb = m % CB;
        constexpr int imm = 16 * s4 * kRow + 256 * (cb / 4);
        cr[m][0] = p2_read_tr<imm>(base + to[0][cb % 4]);
        cr[m][1] = p2_read_tr<imm>(base + to[1][cb % 4]);
      };
      p2_for<0, kPvAhead>(rd);
      p2_for<0, kPvMfma>([&](auto I) __attribute__((always_inline)) {
        constexpr int m = decltype(I)::value, s4 = m / CB, cb = m % CB;
        if constexpr (m + kPvAhead < kPvMfma) {
          rd(std::integral_constant<int, m + kPvAhead>{});
          p2_wait_lgkm<2 * kPvAhead>();
        } else {
          p2_wait_lgkm<2 * (kPvMfma - 1 - m)>();
        }
        p2_tie(cr[m][0]);
        p2_tie(cr[m][1]);
        oacc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cat_bf16x8(cr[m][0], cr[m][1]), pb[s4], oacc[cb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        mid(I);
      });
    };
    auto no_mid = [](auto) {};

    // qkpv(jn, bq, bp, at, mid): tile jn's QK (slots 0 .. kQkReads - 1, one K
    // read each) and the previous tile's PV (the following slots, two C^T
    // reads each) as one stream of MFMAs, with kInFlight LDS reads kept in
    // flight across the boundary between the two products: at about 300 cycles
    // of LDS latency under load, the reads in flight, not the LDS bandwidth,
    // set the rate.  at() runs after the first MFMA (the next tile's DMAs),
    // mid(m) after PV MFMA m (the softmax step).
    constexpr int kSlots = kQkReads + kPvMfma, kReads = kQkReads + 2 * kPvMfma, kInFlight = 12;
    static_assert(kInFlight < 16, "lgkmcnt range");
    auto qkpv = [&](int jn, const lds_u8* bq_p, const lds_u8* bp_p, auto&& at,
                    auto&& mid) __attribute__((always_inline)) {
      const uint32_t bq = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(bq_p));
      const uint32_t bp = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(bp_p));
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) sc[h2] = f32x16_t{};
      sc_tile = jn;  // before the softmax step placed in the PV slots reads it
      p2_u32x4_t kr[kQkReads];
      s16x4_t cr[kPvMfma][2];
      auto rd = [&](auto R) __attribute__((always_inline)) {  // read R of the stream
        constexpr int r = decltype(R)::value;
        if constexpr (r < kQkReads) {
          constexpr int ks = r / 2, h2 = r % 2;
          if constexpr (ks < KS) kr[r] = p2_read16<256 * (ks / 8) + 32 * h2 * kRow>(bq + ko[ks % 8]);
          else kr[r] = p2_read16<32 * h2 * kPeR>(bq + po[ks - KS]);
        } else {
          constexpr int m = (r - kQkReads) / 2, e = (r - kQkReads) % 2, s4 = m / CB, cb = m % CB;
          cr[m][e] = p2_read_tr<16 * s4 * kRow + 256 * (cb / 4)>(bp + to[e][cb % 4]);
        }
      };
      p2_for<0, p2_min<kInFlight, kReads>()>(rd);
      p2_for<0, kSlots>([&](auto I) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value;
        constexpr int done = p2_nreads<kQkReads>(i);  // reads this slot needs complete
        constexpr int before = p2_min<(i == 0 ? 0 : p2_nreads<kQkReads>(i - 1)) + kInFlight, kReads>();
        constexpr int upto = p2_min<done + kInFlight, kReads>();  // reads issued after this slot's issue step
        p2_for<before, upto>(rd);
        p2_wait_lgkm<upto - done>();
        if constexpr (i < kQkReads) {
          constexpr int ks = i / 2, h2 = i % 2;
          p2_tie(kr[i]);
          sc[h2] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kr[i]), qb[ks], sc[h2], 0, 0, 0);
        } else {
          constexpr int m = i - kQkReads, s4 = m / CB, cb = m % CB;
          p2_tie(cr[m][0]);
          p2_tie(cr[m][1]);
          oacc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cat_bf16x8(cr[m][0], cr[m][1]), pb[s4], oacc[cb], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (i == 0) at();
        if constexpr (i >= kQkReads) mid(std::integral_constant<int, i - kQkReads>{});
      });
    };

    // Iteration j < n_tiles - 1 (tile j in buffer j % 3, tile j + 1 in
    // (j + 1) % 3): wait for this wave's DMAs of tile j + 1 and meet at the
    // barrier (tile j + 1 complete, every wave done with iteration j - 1 and so
    // with buffer (j + 2) % 3), start tile j + 2's DMAs into that buffer (past
    // the last tile they re-read its rows: in bounds, never read), then tile
    // j + 1's QK and softmax step with tile j's PV in one region, then the
    // commit.
    auto iter = [&](int j, auto bc) __attribute__((always_inline)) {
      constexpr int C = decltype(bc)::value;
      using N1 = std::integral_constant<int, (C + 1) % 3>;
      using N2 = std::integral_constant<int, (C + 2) % 3>;
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));  // vmcnt(0): this wave's DMAs of tile j + 1 landed
      lds_barrier();
      qkpv(j + 1, buf(N1{}), buf(bc), [&]() __attribute__((always_inline)) { dma_tile(j + 2, buf(N2{})); }, smax_mid);
      commit();
    };
    if (n_tiles > 0) {
      if (flushed) p2_wait_vm<kTileVm + kStores>();  // tile 0's DMAs landed
      else p2_wait_vm<kTileVm>();
      lds_barrier();
      qk(0, buf(I0{}));
      smax();
      commit();
      int j = 0;
      for (; j + 3 < n_tiles; j += 3) {  // block-uniform; unrolled by three for the static buffers
        iter(j, I0{});
        iter(j + 1, I1{});
        iter(j + 2, I2{});
      }
      // the remaining one to three tiles: j .. n_tiles - 1 (tile j in buffer 0)
      if (j + 1 < n_tiles) iter(j, I0{});
      if (j + 2 < n_tiles) iter(j + 1, I1{});
      __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
      lds_barrier();
      const int last = n_tiles - 1 - j;  // 0, 1 or 2
      if (last == 0) pv(buf(I0{}), no_mid);
      else if (last == 1) pv(buf(I1{}), no_mid);
      else pv(buf(I2{}), no_mid);
    }

    if (n_tiles == 0) p2_wait_vm<0>();  // the unused tile copies land before the buffers are reused
    // The output, stored at the next item's start (or after the last item):
    // lane (n, hf) holds channels 32 cb + 8 r4 + 4 hf + {0..3} of its column.
    // A surplus column repeats the block's last query, so its values equal
    // that query's, and it stores them to that query's row.
    const float l_w = l_part + shfl_xor_f32(l_part, 32);
    const float inv = l_w > 0.f ? 1.f / l_w : 0.f;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        pend[cb][r4][0] = pack_bf16x2(oacc[cb][4 * r4] * inv, oacc[cb][4 * r4 + 1] * inv);
        pend[cb][r4][1] = pack_bf16x2(oacc[cb][4 * r4 + 2] * inv, oacc[cb][4 * r4 + 3] * inv);
      }
    pend_op = static_cast<uint16_t*>(a.o_lat) + rq * a.o_rs + head * a.o_hs + 4 * hf;
    pending = true;
    // every wave is done with the LDS buffers before the next item's DMAs
    __syncthreads();
  }
  if (pending) flush();
}

int launch_prefill(const DecodeArgs& a, int dt, int c_dt, hipStream_t s) {
  if (a.n_rows == 0) return 0;
  const int T = a.ad.T;
  constexpr int kQpw = kPrefillQpw, kNw = kPrefillWaves;
  const dim3 grid((T + kNw * kQpw - 1) / (kNw * kQpw), a.n_rows / T), block(kNw * 64);
  // Each wave accumulates all R_pad output channels of its query: built for
  // R_pad <= 256 (larger ranks take the per-row decode path).
  if (a.R > 256) return -1;
  if (dt == 1 && c_dt == 1 && padded_rank(a.R) % 128 == 0) {
    // bf16 cache, latent rows of a multiple of 256 bytes: the 32x32x16 kernel
    // (the same eight query tokens per workgroup, so the same grid)
    static_assert(kP2Waves * kP2Qpw == kNw * kQpw, "query tokens per workgroup");
    // one persistent workgroup per CU (the kernel's LDS takes the CU)
    int dev = 0, n_cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cus < 1)
      return -2;
    const int items = static_cast<int>(grid.x * grid.y);
    const dim3 pgrid(std::min(items, n_cus));
    if (padded_rank(a.R) == 256) hipLaunchKernelGGL(mla_prefill_m32<4>, pgrid, dim3(kP2Waves * 64), 0, s, a);
    else hipLaunchKernelGGL(mla_prefill_m32<2>, pgrid, dim3(kP2Waves * 64), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
  }
  const int rc = with_nb(a.R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value < 4 ? decltype(nb)::value : 4;
    if (dt == 1 && c_dt == 1)
      hipLaunchKernelGGL((mla_prefill_mfma<1, kPrefillDepth, kQpw, kNw, NB>), grid, block, 0, s, a);
    else if (dt == 1 && c_dt == 2)
      hipLaunchKernelGGL((mla_prefill_mfma<2, kPrefillDepth, kQpw, kNw, NB>), grid, block, 0, s, a);
    else return -1;
    return 0;
  });
  if (rc != 0) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace swamla
