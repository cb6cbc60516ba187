// mla_fused.h — the one-token append as the decode kernel folds it in:
// loading a token's inputs, computing its cache row (the same LayerNorm /
// RoPE / e4m3 arithmetic as mla_append_kernel, so the bits are identical)
// and storing it.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mla_args.h"
#include "mla_device.h"
#include "numerics.h"

namespace swamla {

// ---- Fused one-token append inside the decode kernel (bf16 model).
// Inputs of one token as loaded by one wavefront: lane owns latent channels
// NB*lane .. +NB-1 (of the R_pad-channel input row and LayerNorm parameters)
// and (lanes 0..31) the k_pe pair `lane`.  The registers hold the loads'
// words untouched (bf16 pairs for even NB, one zero-extended value per word
// for odd NB): splitting them up at load time would make the wave wait for
// these loads, and so for every load issued before them.
template <int NB>
struct FusedIn {
  static constexpr bool kPair = NB % 2 == 0;
  static constexpr int W = kPair ? NB / 2 : NB;
  uint32_t x[W], wt[W], bs[W];
  uint32_t pe, c, s;
};

// The loads are vm_load()s: the decode kernel's wait for its query (issued
// before the first tile) covers them, and fused_release() follows that wait.
template <int NB>
__device__ __forceinline__ void fused_words(const uint16_t* p, uint32_t (&v)[FusedIn<NB>::W]) {
  if constexpr (FusedIn<NB>::kPair) {
    vm_load<NB / 2>(p, v);
  } else {
#pragma unroll
    for (int i = 0; i < NB; ++i) v[i] = vm_load_u16(p + i);
  }
}

// bf16 bits of the lane's i-th channel
template <int NB>
__device__ __forceinline__ uint32_t fused_half(const uint32_t (&v)[FusedIn<NB>::W], int i) {
  if constexpr (FusedIn<NB>::kPair) return (i & 1) ? (v[i >> 1] >> 16) : (v[i >> 1] & 0xFFFFu);
  else return v[i];
}

template <int NB>
__device__ __forceinline__ FusedIn<NB> fused_load(const AppendArgs& a, int tok, int rope, int lane) {
  const uint16_t* row = static_cast<const uint16_t*>(a.kv_in) + static_cast<int64_t>(tok) * a.in_rs;
  const int pl = lane & (kP / 2 - 1);  // lanes 32..63 repeat pairs 0..31 (unused)
  const int64_t tab = static_cast<int64_t>(rope) * (kP / 2) + pl;
  FusedIn<NB> f;
  fused_words<NB>(row + NB * lane, f.x);
  fused_words<NB>(static_cast<const uint16_t*>(a.ln_w) + NB * lane, f.wt);
  fused_words<NB>(static_cast<const uint16_t*>(a.ln_b) + NB * lane, f.bs);
  uint32_t pe[1];
  vm_load<1>(row + 64 * NB + 2 * pl, pe);
  f.pe = pe[0];
  f.c = vm_load_u16(static_cast<const uint16_t*>(a.cos_tab) + tab);
  f.s = vm_load_u16(static_cast<const uint16_t*>(a.sin_tab) + tab);
  return f;
}

// Release the loaded inputs for use, after a wait that covers their loads:
// each register passes through an empty asm, so no arithmetic on them can be
// scheduled above the point where this is called.
template <int NB>
__device__ __forceinline__ void fused_release(FusedIn<NB>& f) {
#pragma unroll
  for (int i = 0; i < FusedIn<NB>::W; ++i) asm volatile("" : "+v"(f.x[i]), "+v"(f.wt[i]), "+v"(f.bs[i]));
  asm volatile("" : "+v"(f.pe), "+v"(f.c), "+v"(f.s));
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

// Same arithmetic as append_token<1, C_DT, NB> (no loads from memory:
// fused_load read everything; `stage`: ln_stage_bytes<1>() bytes of LDS for
// ln_gather).
template <int C_DT, int NB>
__device__ __forceinline__ FusedTok<C_DT, NB> fused_compute(const FusedIn<NB>& f, float eps, int R, int lane,
                                                            lds_u8* stage) {
  uint32_t xw[(NB + 1) / 2];
#pragma unroll
  for (int i = 0; i < (NB + 1) / 2; ++i)
    xw[i] = fused_half<NB>(f.x, 2 * i) | (2 * i + 1 < NB ? fused_half<NB>(f.x, 2 * i + 1) << 16 : 0u);
  const LnStats st = aten_ln_stats<1>(ln_gather<1, NB>(xw, R, lane, stage), R, eps, lane);
  float x[NB], wt[NB], bs[NB], y[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    x[i] = u2f(fused_half<NB>(f.x, i) << 16);
    wt[i] = u2f(fused_half<NB>(f.wt, i) << 16);
    bs[i] = u2f(fused_half<NB>(f.bs, i) << 16);
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
  t.pe = rope_bf16_packed(u2f(f.pe << 16), u2f(f.pe & 0xFFFF0000u), u2f(f.c << 16), u2f(f.s << 16));
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

}  // namespace swamla
