// mla_kernels.hip — gfx950 kernels for the MLA latent-KV-cache hot path.
//
//   mla_append_*      fused kv_norm LayerNorm + RoPE(k_pe) + optional e4m3
//                     quantisation + scatter into the ragged cache
//                     (reference: models/mla.py:307-323, :409-414)
//   mla_decode_f32    absorbed attention over the latent cache in fp32 on the
//                     VALU, for fp32 models (reference: models/mla.py:417-487)
//   mla_merge_kernel  log-sum-exp merge of split-KV partials
// (the bf16 MFMA decode kernel is in mla_decode.hip, the prefill kernel in
// mla_prefill.hip, shared device code in mla_device.h and mla_fused.h)
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
__device__ __forceinline__ void append_token(const AppendArgs& a, int tok, int lane, lds_u8* stage) {
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
  T xr[NB];
  load_lane<NB>(row + NB * lane, xr);
  constexpr int W = IN_DT == 1 ? (NB + 1) / 2 : NB;
  uint32_t xw[W];
#pragma unroll
  for (int i = 0; i < W; ++i) {
    if constexpr (IN_DT == 1) xw[i] = xr[2 * i] | (2 * i + 1 < NB ? static_cast<uint32_t>(xr[2 * i + 1]) << 16 : 0u);
    else xw[i] = f2u(xr[i]);
  }
  const LnStats st = aten_ln_stats<IN_DT>(ln_gather<IN_DT, NB>(xw, a.R, lane, stage), a.R, a.eps, lane);
  float x[NB], wt[NB], bs[NB], y[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    x[i] = E::ld(xr, i);
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
  __shared__ __attribute__((aligned(16))) uint8_t stage[4 * ln_stage_bytes<IN_DT>()];
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= a.n_tok) return;
  append_token<IN_DT, C_DT, NB>(a, tok, threadIdx.x & 63, (lds_u8*)(stage) + (threadIdx.x >> 6) * ln_stage_bytes<IN_DT>());
}

// ---------------------------------------------------------------------------
// Kernel 1 at prompt sizes: bf16 rows of R_pad = 256 channels, four tokens
// per wavefront, one aligned group of 16 lanes per token (16 tokens per
// block).  Lane l of a group owns latent channels 16 l .. 16 l + 15 (two
// 16-byte loads and stores) and k_pe values 4 l .. 4 l + 3.  The LayerNorm
// statistics are aten_ln_stats on the group: for a bf16 row of at most 256
// channels ATen's vectorised pass has at most 16 Welford streams, one per
// lane of the group, so every lane runs one and the statistics are the same
// arithmetic, bit for bit, as the one-token-per-wavefront kernel's.
// ---------------------------------------------------------------------------
// RC > 0: the kernel for kv_lora_rank RC exactly (the statistics' counts,
// divisions and padding masks fold at compile time); RC = 0: any R.
template <int C_DT, int RC>
__global__ __launch_bounds__(256) void mla_append_g16_kernel(AppendArgs a) {
  constexpr int RP = 256, K = 16;  // channels per lane
  const int R = RC > 0 ? RC : a.R;
  constexpr int kStage = ln_stage_g16_bytes();
  __shared__ __attribute__((aligned(16))) uint8_t stage[16 * kStage];
  const int lane = threadIdx.x & 63, l16 = lane & 15;
  const int slot = threadIdx.x >> 4;  // the block's token
  const int tok = blockIdx.x * 16 + slot;
  if (tok >= a.n_tok) return;  // the whole group
  const TokAddr ta = tok_addr(a.ad, tok);
  const int b = ta.b, pos = ta.pos, rp = ta.rope;
  if (b < 0 || b >= a.cache_b || pos < 0 || pos >= a.cache_s || rp < 0 || rp >= a.rope_len) {
    if (l16 == 0 && a.err_flag) a.err_flag[0] = 1;
    return;
  }
  // the row, the LayerNorm parameters and the rope pairs as packed bf16 words
  const uint16_t* row = static_cast<const uint16_t*>(a.kv_in) + static_cast<int64_t>(tok) * a.in_rs;
  uint32_t xw[K / 2], ww[K / 2], bw[K / 2], pe[2];
  load_lane<K / 2>(reinterpret_cast<const uint32_t*>(row) + (K / 2) * l16, xw);
  load_lane<2>(reinterpret_cast<const uint32_t*>(row + RP) + 2 * l16, pe);
  const LnStats st = aten_ln_stats<1, 16>(
      ln_gather<1, K, 16>(xw, R, l16, (lds_u8*)(stage) + slot * kStage), R, a.eps, lane);
  // The LayerNorm parameters are loaded after the statistics (the compiler
  // would hoist them): fewer registers live across the statistics, 71
  // against 87 VGPRs, measured 43.8 against 47.8 us at 131,072 tokens.
  asm volatile("" ::: "memory");
  load_lane<K / 2>(static_cast<const uint32_t*>(a.ln_w) + (K / 2) * l16, ww);
  load_lane<K / 2>(static_cast<const uint32_t*>(a.ln_b) + (K / 2) * l16, bw);
  // the affine, one channel at a time (channels >= R are padding: 0)
  auto yv = [&](int i) {
    const int h = (i & 1) * 16;
    const float x = u2f((xw[i >> 1] >> h) << 16), w = u2f((ww[i >> 1] >> h) << 16), bb = u2f((bw[i >> 1] >> h) << 16);
    return (RC >= RP || K * l16 + i < R) ? aten_ln_affine<1>(x, w, bb, st) : 0.f;
  };
  // bf16 of each channel (the value a bf16 cache holds; e4m3 encodes it):
  // the hardware's round-to-nearest-even conversion, two channels per
  // instruction (finite values and infinities as f32_to_bf16; a NaN stays a
  // NaN, its payload bits are not kept equal to any other path's)
  uint32_t yw[K / 2];
#pragma unroll
  for (int i = 0; i < K / 2; ++i) yw[i] = pack_bf16x2(yv(2 * i), yv(2 * i + 1));

  const int64_t crow = static_cast<int64_t>(b) * a.cache_s + pos;
  if constexpr (C_DT == 1) {
    store_lane<K / 2>(reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.ckv) + crow * RP) + (K / 2) * l16, yw);
  } else {
    // e4m3 per token: amax over the group's channels, scale = max(amax,
    // 1e-12) / 448, code = RNE(y / scale) of the bf16-rounded channel
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < K / 2; ++i) amax = fmaxf(amax, fmaxf(fabsf(u2f(yw[i] << 16)), fabsf(u2f(yw[i] & 0xFFFF0000u))));
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) amax = fmaxf(amax, shfl_xor_f32(amax, m));
    const float scale = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
    uint32_t cw[K / 4];
#pragma unroll
    for (int q = 0; q < K / 4; ++q) {
      uint32_t c = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * q + e;
        const float yb = u2f((yw[i >> 1] >> ((i & 1) * 16)) << 16);
        c |= static_cast<uint32_t>(f32_to_e4m3(__fdiv_rn(yb, scale))) << (8 * e);
      }
      cw[q] = c;
    }
    store_lane<K / 4>(reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.ckv) + crow * RP) + (K / 4) * l16, cw);
    if (l16 == 0) a.ckv_scale[crow] = scale;
  }

  // RoPE on k_pe: the lane's pairs 2 l16 and 2 l16 + 1
  const uint32_t cw = static_cast<const uint32_t*>(a.cos_tab)[static_cast<int64_t>(rp) * (kP / 4) + l16];
  const uint32_t sw = static_cast<const uint32_t*>(a.sin_tab)[static_cast<int64_t>(rp) * (kP / 4) + l16];
  uint32_t ow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    ow[j] = rope_bf16_packed(bf16_to_f32(pe[j] & 0xFFFF), bf16_to_f32(pe[j] >> 16),
                             bf16_to_f32(j ? cw >> 16 : cw & 0xFFFF), bf16_to_f32(j ? sw >> 16 : sw & 0xFFFF));
  }
  store_lane<2>(reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.kpe) + crow * kP) + 2 * l16, ow);
}

// ---------------------------------------------------------------------------
// Kernel 2 on the VALU in fp32: fp32 models (any rank), and bf16 models at
// ranks above the MFMA kernel's 512 (up to 1024).  One block of 256 threads
// per (row, split); 16-token tiles staged in LDS as fp32 (bf16 values
// widened, e4m3 codes times the token's scale).  DT: model dtype (queries,
// RoPE tables, k_pe cache, output: 0 fp32 / 1 bf16, whose q_pe rotation
// rounds every product and sum to bf16 as the MFMA kernels' does); C_DT:
// latent cache (0 fp32 / 1 bf16 / 2 e4m3).
// ---------------------------------------------------------------------------
template <int DT, int C_DT, int NB>
__global__ __launch_bounds__(256) void mla_decode_vec(DecodeArgs a) {
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
  if (a.balance > 0) {  // as in mla_decode_dma
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
  using E = Elem<DT>;
  using T = typename E::T;
  const T* qa = static_cast<const T*>(a.q_abs) + r * a.qa_rs;
  const T* qp = static_cast<const T*>(a.q_pe) + r * a.qp_rs;
  const T* ct = static_cast<const T*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
  const T* st = static_cast<const T*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
  for (int i = t; i < kH * RP; i += 256) {
    const int h = i / RP, c = i % RP;
    q_s[h][c] = c < a.R ? E::ld(qa, h * a.qa_hs + c) : 0.f;  // the padding channels are zero
  }
  for (int i = t; i < kH * kP / 2; i += 256) {
    const int h = i / (kP / 2), pi = i % (kP / 2);
    float o1, o2;
    rope_pair<DT>(E::ld(qp, h * a.qp_hs + 2 * pi), E::ld(qp, h * a.qp_hs + 2 * pi + 1), E::ld(ct, pi), E::ld(st, pi),
                  o1, o2);
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

  const T* kpe = static_cast<const T*>(a.kpe);
  auto latent = [&](int64_t row, int c) -> float {
    if constexpr (C_DT == 0) return static_cast<const float*>(a.ckv)[row * RP + c];
    else if constexpr (C_DT == 1) return bf16_to_f32(static_cast<const uint16_t*>(a.ckv)[row * RP + c]);
    else return e4m3_to_f32(static_cast<const uint8_t*>(a.ckv)[row * RP + c]) * a.ckv_scale[row];
  };
  for (int base = t0; base < t1; base += TT) {
    __syncthreads();
    for (int i = t; i < TT * KC; i += 256) {
      const int j = i / KC, c = i % KC;
      const int tok = base + j;
      float v = 0.f;
      if (tok < t1) v = c < RP ? latent(row0 + tok, c) : E::ld(kpe, (row0 + tok) * kP + (c - RP));
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
    T* op = static_cast<T*>(a.o_lat) + r * a.o_rs + h_pv * a.o_hs + c_pv;
#pragma unroll
    for (int jj = 0; jj < CPV; ++jj) op[jj] = E::from_f32(o[jj] * inv);
    if (a.lse_out && (t & 15) == 0)
      a.lse_out[static_cast<int64_t>(r) * kH + h_pv] = (Lh > 0.f) ? (m_s[h_pv] + __log2f(Lh)) * kLn2 : -INFINITY;
    return;
  }
  const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + h_pv;
  float* op = a.o_part + pidx * RP + c_pv;
#pragma unroll
  for (int jj = 0; jj < CPV; ++jj) op[jj] = o[jj] * inv;
  if ((t & 15) == 0) a.lse_part[pidx] = (Lh > 0.f) ? (m_s[h_pv] + __log2f(Lh)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Kernel 3: split-KV merge, one wavefront per (row r, head h):
//   o = sum_s exp(lse_s - M) o_s / sum_s exp(lse_s - M),  M = max_s lse_s
// The statistics are wavefront reductions: lane l takes splits l, l + 64, ...,
// M is the wave max of their log-sum-exps, each lane forms its splits'
// weights once and their sum is a wave sum.  The weighted sum of the partial
// rows then runs over the splits in order (lane: 4 channels of each
// 256-channel chunk; TWO: the padded row, at most 512 channels, spans a
// second chunk), split s's weight broadcast from lane s % 64 (readlane).
// The partial rows' loads go out 8 splits at a time.  Latency: the row's
// length, lane l's log-sum-exp and the first 8 partial rows are all issued
// before the row's split count is known (slots past the count, up to
// n_splits - 1, are in the buffers but may hold stale, even non-finite,
// values: they are dropped by selects, never multiplied in).  An empty split
// (lse -inf) has weight 0; rows of at most one split were written by the
// decode kernel itself.
// ---------------------------------------------------------------------------
template <int DT, int CH>
__global__ __launch_bounds__(64) void mla_merge_kernel(MergeArgs a) {
  // CH chunks of 256 channels (R_pad <= 256 CH): lane l reads channels 4 l ..
  // 4 l + 3 of each
  const int h = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
  const int rp = 64 * ((a.R + 63) / 64);
  const int64_t base = static_cast<int64_t>(r) * a.n_splits * a.H + h;  // (row, split 0, head) slot
  const int plan = a.plan ? *a.plan : 0;
  const int L = clamped_row_len(a.ad, r, a.cache_b, a.cache_s);
  const int last = a.n_splits - 1;
  const float le = a.lse_part[base + static_cast<int64_t>(min(lane, last)) * a.H];
  // channels read: a lane past the row re-reads channel 0 (its sums are not stored)
  int cr_[CH];
  bool on_[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    on_[k] = 4 * lane + 256 * k < rp;
    cr_[k] = on_[k] ? 4 * lane + 256 * k : 0;
  }
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 v[CH][8];
  auto load_group = [&](int g, int s_max) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float* p = a.o_part + (base + static_cast<int64_t>(min(g + j, s_max)) * a.H) * rp;
#pragma unroll
      for (int k = 0; k < CH; ++k) v[k][j] = *reinterpret_cast<const float4*>(p + cr_[k]);
    }
  };
  load_group(0, last);
  // at most n_splits (a plan word from another launch cannot send the reads
  // past the row's slots)
  const int ns = min(row_splits(L, a.n_splits, a.min_chunk, plan).ns, a.n_splits);
  if (ns <= 1) return;

  auto lse_of = [&](int s) { return s < ns ? a.lse_part[base + static_cast<int64_t>(s) * a.H] : -INFINITY; };
  const float l0 = lane < ns ? le : -INFINITY;
  float M = l0;
  for (int s = lane + 64; s < ns; s += 64) M = fmaxf(M, lse_of(s));
  M = lane_group_max<64>(M);
  // all splits empty: M = -inf, every weight 0, output 0 and lse -inf
  const float w0 = l0 == -INFINITY ? 0.f : __expf(l0 - M);
  float tot = w0;
  for (int s = lane + 64; s < ns; s += 64) {
    const float l = lse_of(s);
    tot += l == -INFINITY ? 0.f : __expf(l - M);
  }
  tot = lane_group_sum<64>(tot);
  const float inv = tot > 0.f ? 1.f / tot : 0.f;

  float4 acc[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) acc[k] = z;
  float wl = w0;  // weight of split (g & ~63) + lane
  for (int g = 0; g < ns; g += 8) {
    if (g > 0) {
      load_group(g, ns - 1);
      if ((g & 63) == 0) {
        const float l = lse_of(g + lane);
        wl = l == -INFINITY ? 0.f : __expf(l - M);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool in = g + j < ns;  // uniform
      const float wj = u2f(__builtin_amdgcn_readlane(f2u(wl), (g & 63) + j));
      if (in) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          acc[k].x += wj * v[k][j].x;
          acc[k].y += wj * v[k][j].y;
          acc[k].z += wj * v[k][j].z;
          acc[k].w += wj * v[k][j].w;
        }
      }
    }
  }
  auto store = [&](int c, const float4& ac) {
    if constexpr (DT == 0) {
      float* op = static_cast<float*>(a.o_lat) + r * a.o_rs + h * a.o_hs;
      *reinterpret_cast<float4*>(op + c) = make_float4(ac.x * inv, ac.y * inv, ac.z * inv, ac.w * inv);
    } else {
      uint16_t* op = static_cast<uint16_t*>(a.o_lat) + r * a.o_rs + h * a.o_hs;
      uint2 pk;
      pk.x = f32_to_bf16(ac.x * inv) | (static_cast<uint32_t>(f32_to_bf16(ac.y * inv)) << 16);
      pk.y = f32_to_bf16(ac.z * inv) | (static_cast<uint32_t>(f32_to_bf16(ac.w * inv)) << 16);
      *reinterpret_cast<uint2*>(op + c) = pk;
    }
  };
#pragma unroll
  for (int k = 0; k < CH; ++k)
    if (on_[k]) store(4 * lane + 256 * k, acc[k]);
  if (a.lse_out && lane == 0) a.lse_out[static_cast<int64_t>(r) * a.H + h] = M + __logf(tot);
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
  // bf16 rows of 256 padded channels whose vectors are 16-byte aligned: four
  // tokens per wavefront
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (in_dt == 1 && (c_dt == 1 || c_dt == 2) && padded_rank(a.R) == 256 && a16(a.kv_in) && a.in_rs % 8 == 0 &&
      a16(a.ln_w) && a16(a.ln_b) && (reinterpret_cast<uintptr_t>(a.cos_tab) & 3) == 0 &&
      (reinterpret_cast<uintptr_t>(a.sin_tab) & 3) == 0) {
    const dim3 g16((a.n_tok + 15) / 16);
    if (a.R == 256) {
      if (c_dt == 1) hipLaunchKernelGGL((mla_append_g16_kernel<1, 256>), g16, block, 0, s, a);
      else hipLaunchKernelGGL((mla_append_g16_kernel<2, 256>), g16, block, 0, s, a);
    } else {
      if (c_dt == 1) hipLaunchKernelGGL((mla_append_g16_kernel<1, 0>), g16, block, 0, s, a);
      else hipLaunchKernelGGL((mla_append_g16_kernel<2, 0>), g16, block, 0, s, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
  }
  const int rc = with_nb_wide(a.R, [&](auto nb) {
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

// The fp32 decode kernel (fp32 models); the MFMA kernel's launcher in
// mla_decode.hip dispatches here for them.
namespace {
// The VALU decode instance: fp32 models with an fp32 cache at any rank; bf16
// models with a bf16 or e4m3 cache at ranks above kMaxNB (the MFMA kernel
// takes the others).
template <int NB>
const void* decode_vec_kernel(int dt, int c_dt) {
  if (dt == 0 && c_dt == 0) return reinterpret_cast<const void*>(&mla_decode_vec<0, 0, NB>);
  if constexpr (NB > kMaxNB) {
    if (dt == 1 && c_dt == 1) return reinterpret_cast<const void*>(&mla_decode_vec<1, 1, NB>);
    if (dt == 1 && c_dt == 2) return reinterpret_cast<const void*>(&mla_decode_vec<1, 2, NB>);
  }
  return nullptr;
}
}  // namespace

int launch_decode_vec(const DecodeArgs& a, int dt, int c_dt, hipStream_t s) {
  const dim3 grid = a.balance > 0 ? dim3(a.balance, 1) : dim3(a.n_splits, a.n_rows);
  const int rc = with_nb_wide(a.R, [&](auto nb) {
    const void* fn = decode_vec_kernel<decltype(nb)::value>(dt, c_dt);
    if (!fn) return -1;
    void* args[] = {const_cast<DecodeArgs*>(&a)};
    return hipLaunchKernel(fn, grid, dim3(256), args, 0, s) == hipSuccess ? 0 : -2;
  });
  if (rc != 0) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int decode_vec_blocks_per_cu(int dt, int c_dt, int R, int* blocks) {
  return with_nb_wide(R, [&](auto nb) {
    const void* fn = decode_vec_kernel<decltype(nb)::value>(dt, c_dt);
    if (!fn) return -1;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, 256, 0) != hipSuccess || n < 1) return -2;
    *blocks = 1;  // the split plan deals one block per CU
    return 0;
  });
}

int launch_merge(const MergeArgs& a, int dt, hipStream_t s) {
  if (a.n_rows == 0 || a.n_splits <= 1) return 0;
  const dim3 grid(a.H, a.n_rows), block(64);
  const int ch = (padded_rank(a.R) + 255) / 256;  // 256-channel chunks of the padded row
  if (dt != 0 && dt != 1) return -1;
  if (ch == 1) {
    if (dt == 1) hipLaunchKernelGGL((mla_merge_kernel<1, 1>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((mla_merge_kernel<0, 1>), grid, block, 0, s, a);
  } else if (ch == 2) {
    if (dt == 1) hipLaunchKernelGGL((mla_merge_kernel<1, 2>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((mla_merge_kernel<0, 2>), grid, block, 0, s, a);
  } else if (ch <= 4) {
    if (dt == 1) hipLaunchKernelGGL((mla_merge_kernel<1, 4>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((mla_merge_kernel<0, 4>), grid, block, 0, s, a);
  } else {
    return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace swamla
