// mla_prefill.hip — gfx950 attention of a prefill chunk over the latent
// cache (reference: models/mla.py:417-487 with seqlen > 1).
#include <hip/hip_runtime.h>
#include <stdint.h>

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
        float o1, o2;
        rope_pair<1>(bf16_to_f32(wv_in[jj] & 0xFFFF), bf16_to_f32(wv_in[jj] >> 16), bf16_to_f32(cj),
                     bf16_to_f32(sj), o1, o2);
        wv[jj] = f32_to_bf16(o1) | (static_cast<uint32_t>(f32_to_bf16(o2)) << 16);
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


int launch_prefill(const DecodeArgs& a, int dt, int c_dt, hipStream_t s) {
  if (a.n_rows == 0) return 0;
  const int T = a.ad.T;
  constexpr int kQpw = kPrefillQpw, kNw = kPrefillWaves;
  const dim3 grid((T + kNw * kQpw - 1) / (kNw * kQpw), a.n_rows / T), block(kNw * 64);
  // Each wave accumulates all R_pad output channels of its query: built for
  // R_pad <= 256 (larger ranks take the per-row decode path).
  if (a.R > 256) return -1;
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
