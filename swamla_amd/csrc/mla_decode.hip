// mla_decode.hip — absorbed decode attention over the latent cache on gfx950
// (bf16 model, bf16 or e4m3 cache), with the one-token append optionally
// folded in.  Reference: models/mla.py:417-487 (cache gather, wkv_b
// up-projection, SDPA), re-associated: s_t = scale (q_abs . c_t + q_pe . k_pe_t),
// o_lat = sum_t softmax(s)_t c_t; with the fused append also :307-323, :409-414.
//
// One workgroup of four wavefronts per (query row, split).  The split's tokens
// are cut into 16-token sub-tiles dealt round-robin to the waves (a short first
// round of n_sub % 4 sub-tiles, then full rounds in which the four waves cover
// 64 consecutive tokens; the last sub-tile lands on a least-loaded wave), and
// every wave runs its own online softmax over its sub-tiles: no barrier or
// exchange inside the loop.  Per sub-tile a wave
//   * streams the 16 latent rows and 16 rope rows from HBM straight into its
//     own LDS ring buffer with global_load_lds_dwordx4 (1 KB per instruction,
//     whole 128-byte lines, non-temporal), NBUF sub-tiles in flight;
//     16-byte chunks are XOR-swizzled within each 128-byte group of a row so
//     that the operand reads below hit distinct banks;
//   * S^T[16 tok x 16 heads] = K . Q^T: mfma_f32_16x16x32_bf16, K from LDS
//     (16 tokens x 8 channels per instruction), Q^T in registers for the
//     whole split;
//   * per-head maxima over the sub-tile with two row-swap permutes, lazily
//     moved softmax reference (log2 domain);
//   * O^T[16 ch x 16 heads] += C^T . P^T per 16-channel block:
//     mfma_f32_16x16x16_bf16 with C^T read transposed from LDS
//     (ds_read_b64_tr_b16) and P^T straight from the score registers (the
//     score accumulator's layout is the product's B operand).
// An e4m3 cache is streamed as codes and decoded exactly (packed
// cvt_scalef32_pk_bf16_fp8 at scale 1) into a per-wave bf16 staging tile;
// its per-token scale multiplies the latent score and the token's weight.
// At the end the four waves' (max, sum, O) meet in LDS and are combined in a
// fixed order; a one-split row writes o_lat (and its log-sum-exp if asked),
// otherwise the split writes fp32 partials and a natural-log LSE for the merge.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "mla_args.h"
#include "mla_device.h"
#include "mla_fused.h"
#include "mla_plan.h"
#include "numerics.h"

namespace swamla {

int launch_decode_vec(const DecodeArgs& a, int dt, int c_dt, hipStream_t s);
int decode_vec_blocks_per_cu(int dt, int c_dt, int R, int* blocks);

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kSubTok = 16;   // tokens per wave sub-tile
constexpr int kDecWaves = 4;  // waves per workgroup
constexpr int kLdsMax = 160 * 1024;

// Chunk swizzles for gfx950's LDS (64 banks of 4 bytes: a 16-byte-per-lane
// read serves 16 lanes per cycle from one 256-byte window, an 8-byte read 32
// lanes).  16-byte chunk c of latent row t (a sub-tile's 16 rows) lives at
// c ^ swz<NB>(t); rope row t's at c ^ swp(t).  The XOR stays inside aligned
// groups of kSwG chunks, which divide the row.
//  * rows of a multiple of 256 bytes (NB even): 16-chunk groups, swz = (2t |
//    t >> 3) & 15.  The K read of one chunk from all 16 rows hits 16 distinct
//    slots of a window; the transposed C^T read (4 rows x 32 bytes per 16
//    lanes) puts rows 0..7 on the 8 even slot pairs, rows 8..15 on the odd.
//  * rows of an odd multiple of 128 bytes (NB odd; consecutive rows alternate
//    window halves): 8-chunk groups, swz = ((t & 14) | t >> 3) & 7: each
//    parity's 8 rows take distinct slots, and the transposed read's rows
//    distinct slot pairs.
//  * rope rows (128 bytes): swp = t >> 1 (each parity's rows distinct).
template <int NB>
constexpr int kSwG = NB % 2 == 0 ? 16 : 8;
template <int NB>
__device__ __forceinline__ int swz(int t) {
  if constexpr (NB % 2 == 0) return ((t << 1) | (t >> 3)) & 15;
  else return ((t & 14) | (t >> 3)) & 7;
}
__device__ __forceinline__ int swp(int t) { return (t >> 1) & 7; }

constexpr int cmin(int a, int b) { return a < b ? a : b; }
constexpr int cmax(int a, int b) { return a > b ? a : b; }

// Geometry of one instance (cache dtype, R_pad = 64 NB, HG head groups of 16
// heads, all served by each of the workgroup's four waves).
template <int C_DT, int NB, int HG = 1>
struct DecGeo {
  static constexpr int RP = 64 * NB;
  static constexpr int kLat = C_DT == 2 ? kSubTok * RP : kSubTok * 2 * RP;  // latent bytes of a sub-tile
  static constexpr int kPe = kSubTok * 2 * kP;                                // 2 KB of rope rows
  static constexpr int kSc = C_DT == 2 ? 256 : 0;                             // e4m3 scales (4 copies of 16)
  static constexpr int kSub = kLat + kPe + kSc;
  static constexpr int kStage = C_DT == 2 ? kSubTok * 2 * RP : 0;            // e4m3: decoded bf16 tile
  static constexpr int kVm = (kLat + kPe) / 1024 + (C_DT == 2 ? 1 : 0);      // vm operations per sub-tile
  // The ring: kFill sub-tiles are issued ahead of the loop; while one is
  // processed, at most kCap more are in flight.  Fewer bytes in flight stream
  // faster here: 2 and 2 (three buffers) against 3 and 3 (four buffers)
  // measured 18.1 against 18.4-18.9 us per config-2 launch, and 89.9
  // against 90.6-91.1 us at config 5 (e4m3).
  static constexpr int kWavesWG = kDecWaves;
  static constexpr int kFillWant = 2, kCapWant = 2;
  static constexpr int NBUF =
      cmin(cmin(cmax(kCapWant + 1, kFillWant), (kLdsMax / kWavesWG - kStage) / kSub), 63 / kVm + 1);
  static constexpr int kCap = cmin(kCapWant, NBUF - 1);
  static constexpr int kFill = cmin(kFillWant, NBUF);
  // The fused append's LayerNorm stages its row in a ring buffer the fill
  // leaves free, else in an area of its own.
  static constexpr int kLnOwn = kFill == NBUF ? ln_stage_bytes<1>() : 0;
  // epilogue: each wave stashes, in its own LDS area, per head group and head
  // a row of RP fp32 (+4 pad), then its max / l / e per head
  static constexpr int kCombRow = RP + 4;
  static constexpr int kStashG = kH * kCombRow + 3 * kH;  // floats per head group
  static constexpr int kStash = HG * kStashG * 4;
  static constexpr int kRing = NBUF * kSub + kStage + kLnOwn;
  static constexpr int kWave = cmax(kRing, kStash);  // LDS bytes per wave
  static constexpr int kLds = kWavesWG * kWave;
  static_assert(NBUF >= 2, "a sub-tile ring needs two buffers");
  static_assert(ln_stage_bytes<1>() <= kSub, "the fused LayerNorm stages its row in a ring buffer");
  static_assert(kCap >= 1 && kFill >= 1 && kCap <= NBUF - 1, "ring depth");
  static_assert(kLds <= kLdsMax, "LDS budget");
};

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt / lgkmcnt not waited for).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Wait until at most `ahead` sub-tiles (of V vm operations each) are in flight.
template <int V, int NBUF>
__device__ __forceinline__ void wait_subtiles(int ahead) {
  static_assert(NBUF <= 5, "extend the cases");
  if constexpr (NBUF > 4) if (ahead >= 4) { wait_vm<4 * V>(); return; }
  if constexpr (NBUF > 3) if (ahead >= 3) { wait_vm<3 * V>(); return; }
  if constexpr (NBUF > 2) if (ahead >= 2) { wait_vm<2 * V>(); return; }
  if (ahead >= 1) { wait_vm<V>(); return; }
  wait_vm<0>();
}

// 16 (4) bytes per lane from global memory into LDS at dst + 16 (4) * lane,
// non-temporal (aux 2): the cache is streamed once.
__device__ __forceinline__ void dma16(const void* src, lds_u8* dst) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<lds_void*>(dst), 16, 0, 2);
}
__device__ __forceinline__ void dma4(const void* src, lds_u8* dst) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<lds_void*>(dst), 4, 0, 2);
}

template <typename T>
__device__ __forceinline__ void lds_st(lds_u8* p, const T& v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>(p) = v;
}
typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void lds_st16(lds_u8* p, uint4 v) {
  *reinterpret_cast<__attribute__((address_space(3))) u32x4v_t*>(p) = u32x4v_t{v.x, v.y, v.z, v.w};
}
// LDS byte address of an LDS pointer (32 bits on the device).
__device__ __forceinline__ uint32_t lds_off(const lds_u8* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Reads of the streamed tiles.  The compiler cannot tell an LDS read of one
// ring buffer from the DMA still filling another, and would drain every load
// in flight (s_waitcnt vmcnt(0)) before each LDS read; these reads are
// therefore issued as inline assembly after the explicit vmcnt wait for the
// buffer they read, and their results are released by lds_fence(): one
// s_waitcnt lgkmcnt(0), then an empty asm that redefines each result so no
// use can be scheduled above the wait.
template <int OFF>
__device__ __forceinline__ u32x4v_t ds_read16(uint32_t addr) {
  u32x4v_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <int OFF>
__device__ __forceinline__ s16x4_t ds_read8(uint32_t addr) {
  s16x4_t v;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <int OFF>
__device__ __forceinline__ s16x4_t ds_read_tr16(uint32_t addr) {
  s16x4_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <typename T>
__device__ __forceinline__ void tie(T& v) { asm volatile("" : "+v"(v)); }

// Compile-time loop: f(std::integral_constant<int, I>) for I = 0 .. N-1.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// One wave's share of a split's sub-tile stream.  The split [t0, t1) is cut
// into n_sub 16-token sub-tiles dealt to the four waves: a short first round
// deals sub-tiles 0 .. rem - 1 (rem = n_sub % 4) to waves 0 .. rem - 1, then
// full rounds follow: wave w's k-th sub-tile is w (w < rem, k = 0), else
// rem + w + 4 (k - [w < rem]).  So the split's last sub-tile goes to wave 3,
// one of the waves with the fewest sub-tiles.  issue(k) streams the wave's
// k-th sub-tile (16 latent rows, 16 rope rows, e4m3: 16 scales) from HBM into
// ring buffer k % NBUF of the wave's LDS with G::kVm vector-memory
// instructions: bf16 rows with their 16-byte chunks swizzled (slot s of row
// tt holds chunk s ^ swz(tt), rope rows ^ swp(tt)), e4m3 code rows as they
// lie.  A sub-tile past the split's end re-reads its last row (in bounds).
template <int C_DT, int NB, int HG = 1>
struct SubStream {
  using G = DecGeo<C_DT, NB, HG>;
  static constexpr int kLatQ = G::kLat / 1024;
  static constexpr int kLatRow = C_DT == 2 ? G::RP : 2 * G::RP;  // bytes of a latent cache row
  int t0, t_last, rem, my_n, j_base, w;
  int64_t row0;
  const uint8_t* ckv;
  const uint8_t* kpe;
  const float* scale;
  lds_u8* wave_lds;
  // per-lane source offsets within a sub-tile (16 rows from its first
  // token) for each DMA instruction
  uint32_t lat_off[kLatQ], pe_off[2];

  __device__ __forceinline__ SubStream(int t0_, int t1, int w_, int lane, int64_t row0_, const void* ckv_,
                                       const void* kpe_, const float* scale_, lds_u8* wave_lds_)
      : t0(t0_), w(w_), row0(row0_), ckv(static_cast<const uint8_t*>(ckv_)),
        kpe(static_cast<const uint8_t*>(kpe_)), scale(scale_), wave_lds(wave_lds_) {
    const int n_sub = t1 > t0 ? (t1 - t0 + kSubTok - 1) / kSubTok : 0;
    rem = n_sub % kDecWaves;
    my_n = n_sub / kDecWaves + (w < rem ? 1 : 0);
    j_base = rem + w - (w < rem ? kDecWaves : 0);  // j = j_base + 4 k, except (w < rem, k = 0): j = w
    t_last = t1 > 0 ? t1 - 1 : 0;
#pragma unroll
    for (int q = 0; q < kLatQ; ++q) {
      const int o = 1024 * q + 16 * lane;
      if constexpr (C_DT == 2) {
        lat_off[q] = o;
      } else {
        const int tt = o / (2 * G::RP), sl = (o % (2 * G::RP)) >> 4;
        lat_off[q] = tt * (2 * G::RP) + 16 * (sl ^ swz<NB>(tt));
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int tt = 8 * q + (lane >> 3);
      pe_off[q] = tt * (2 * kP) + 16 * ((lane & 7) ^ swp(tt));
    }
  }
  __device__ __forceinline__ int sub_of(int k) const { return (k == 0 && w < rem) ? w : j_base + kDecWaves * k; }
  __device__ __forceinline__ void issue(int k, int lane) const {
    const int tb = t0 + kSubTok * sub_of(k);
    lds_u8* const dst = wave_lds + (k % G::NBUF) * G::kSub;
    if (tb + kSubTok - 1 <= t_last) {  // uniform: the whole sub-tile is in the split
      const uint8_t* lb = ckv + (row0 + tb) * kLatRow;
      const uint8_t* pb = kpe + (row0 + tb) * (2 * kP);
#pragma unroll
      for (int q = 0; q < kLatQ; ++q) dma16(lb + lat_off[q], dst + 1024 * q);
#pragma unroll
      for (int q = 0; q < 2; ++q) dma16(pb + pe_off[q], dst + G::kLat + 1024 * q);
      if constexpr (C_DT == 2) dma4(scale + row0 + tb + (lane & 15), dst + G::kLat + G::kPe);
      return;
    }
    // the split's last, partial sub-tile: rows past its end re-read its last row
#pragma unroll
    for (int q = 0; q < kLatQ; ++q) {
      const int tt = (1024 * q + 16 * lane) / kLatRow;
      const int tok = min(tb + tt, t_last);
      dma16(ckv + (row0 + tok) * kLatRow + (lat_off[q] - tt * kLatRow), dst + 1024 * q);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int tt = 8 * q + (lane >> 3);
      const int tok = min(tb + tt, t_last);
      dma16(kpe + (row0 + tok) * (2 * kP) + (pe_off[q] - tt * (2 * kP)), dst + G::kLat + 1024 * q);
    }
    if constexpr (C_DT == 2) {
      const int tok = min(tb + (lane & 15), t_last);
      dma4(scale + row0 + tok, dst + G::kLat + G::kPe);
    }
  }
};

}  // namespace

template <int C_DT, bool FUSE, int NB, int HG>
__global__ __launch_bounds__(kDecWaves * 64, 1) void mla_decode_dma(DecodeArgs a) {
  using G = DecGeo<C_DT, NB, HG>;
  constexpr int RP = G::RP, NBUF = G::NBUF;
  constexpr int HT = kH * HG;  // heads of the launch
  __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[G::kLds];
  lds_u8* const lds = (lds_u8*)(lds_raw);  // the LDS address space, for the DMA and typed LDS access

  // Each wave serves all HG head groups (heads 16 hg .. 16 hg + 15) from one
  // stream of its sub-tiles: every operand read from LDS feeds one MFMA per
  // head group, and each head group runs its own online softmax.
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave of the workgroup
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  if constexpr (FUSE) {
    // The fused append's own arguments come in with the rest at entry: read
    // first inside the owning wave's branch, they sit on kernel-argument lines
    // no other wave touches, and that cold read would hold back the wave's
    // first tile.
    asm volatile("" ::"s"(a.fa.in_rs), "s"(a.fa.ln_w), "s"(a.fa.ln_b), "s"(a.fa.kv_in));
  }

  // ---- workgroup -> (row, split)
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
    ra = bs.addr;
  } else {
    ra = row_addr(a.ad, r);
  }

  // ---- query loads (Q^T as the B operand: lane holds head n, 8 channels at
  // 32 kb + 8 g); issued before anything waits.  These and the other loads
  // ahead of the first tile are vm_load()s, released after the explicit wait
  // below.
  uint32_t qraw[HG][2 * NB][4], praw[HG][2][4];
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
    const uint16_t* qa = static_cast<const uint16_t*>(a.q_abs) + r * a.qa_rs + (kH * hg + n) * a.qa_hs;
#pragma unroll
    for (int s = 0; s < 2 * NB; ++s) vm_load<4>(qa + 32 * s + 8 * g, qraw[hg][s]);
  }
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q_pe) + r * a.qp_rs + (kH * hg + n) * a.qp_hs;
#pragma unroll
    for (int s = 0; s < 2; ++s) vm_load<4>(qp + 32 * s + 8 * g, praw[hg][s]);
  }

  const int b = ra.b;
  int L = ra.pos;
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const RowSplits rsp = row_splits(L, a.n_splits, a.min_chunk, bal_chunk);
  const int ns = rsp.ns;
  if (split >= ns && !(ns == 0 && split == 0)) return;
  // Splits run last-first over blockIdx.x: the row's last split, the one that
  // also appends the new token, gets the first workgroup id of the row and so
  // the earliest start (workgroups are dealt to the XCDs in id order, and the
  // later XCDs begin later).
  if (a.balance <= 0 && ns > 0) split = ns - 1 - split;
  const int t0 = split * rsp.chunk;  // a multiple of 16
  const int t1 = min(L, t0 + rsp.chunk);
  const int64_t row0 = static_cast<int64_t>((b < 0 || b >= a.cache_b) ? 0 : b) * a.cache_s;

  // ---- this wave's sub-tiles; wave w's k-th goes to ring buffer k % NBUF
  lds_u8* const wave_lds = lds + w * G::kWave;
  lds_u8* const stage = wave_lds + NBUF * G::kSub;  // e4m3 only
  const SubStream<C_DT, NB, HG> ss(t0, t1, w, lane, row0, a.ckv, a.kpe, a.ckv_scale, wave_lds);
  const int rem = ss.rem, my_n = ss.my_n;
  auto sub_of = [&](int k) { return ss.sub_of(k); };
  auto issue = [&](int k) { ss.issue(k, lane); };

  // The ring fills at once: the first sub-tile right behind the query loads,
  // then (after the RoPE-row and fused-append loads) the next ones.  Every
  // wave issues all kFill of them, also past its own sub-tiles (they then
  // re-read the split's last row, in bounds), so one fixed wait below covers
  // the loads issued before the second.
  issue(0);

  // RoPE row of the query (cos / sin loads go out before the later tiles')
  int rp = ra.rope;
  rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
  const uint16_t* ct = static_cast<const uint16_t*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2);
  const uint16_t* st = static_cast<const uint16_t*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2);
  uint32_t cr[2][2], sr[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    vm_load<2>(ct + (32 * s + 8 * g) / 2, cr[s]);
    vm_load<2>(st + (32 * s + 8 * g) / 2, sr[s]);
  }

  // ---- fused append: the split holding position L - 1 owns the new token
  bool fa_own = false;  // workgroup-uniform
  int fa_k = 0, fa_t = 0, fa_w = 0;
  TokAddr fa_a{0, 0, 0};
  if constexpr (FUSE) {
    if (split == (ns > 0 ? ns - 1 : 0)) {
      fa_a = TokAddr{ra.b, ra.pos - 1, ra.rope};
      if (fa_a.b < 0 || fa_a.b >= a.fa.cache_b || fa_a.pos < 0 || fa_a.pos >= a.fa.cache_s || fa_a.rope < 0 ||
          fa_a.rope >= a.fa.rope_len) {
        if (threadIdx.x == 0 && a.fa.err_flag) a.fa.err_flag[0] = 1;  // skipped, as mla_append does
      } else {
        fa_own = true;  // then L = pos + 1 <= cache_s and t1 = L
        const int j = (fa_a.pos - t0) / kSubTok;
        if (j < rem) {
          fa_w = j;
          fa_k = 0;
        } else {
          fa_w = (j - rem) % kDecWaves;
          fa_k = (j - rem) / kDecWaves + (fa_w < rem ? 1 : 0);
        }
        fa_t = (fa_a.pos - t0) % kSubTok;
      }
    }
  }
  // the wave holding the new token's sub-tile
  const bool fa_wave = FUSE && fa_own && w == fa_w;  // wave-uniform
  FusedIn<NB> fin;
  if constexpr (FUSE)
    if (fa_wave) fin = fused_load<NB>(a.fa, r, fa_a.rope, lane);

#pragma unroll
  for (int k = 1; k < G::kFill; ++k) issue(k);

  bf16x8_t qb[HG][2 * NB + 2];  // Q^T, set once the query has landed
  f32x4_t oacc[HG][4 * NB];
  float m_run[HG], l_part[HG], e_part[HG];
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
    for (int i = 0; i < 4 * NB; ++i) oacc[hg][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_run[hg] = -INFINITY;
    l_part[hg] = 0.f;
    e_part[hg] = 0.f;
  }
  FusedTok<C_DT, NB> ftok;

  // Operand addresses within a sub-tile (bytes), K = kSwG chunks per swizzle
  // group.  QK (A = K): lane (n, g) reads latent row n, chunk (4 s + g) ^ sw,
  // sw = swz(n): a base per s % (K / 4) plus 16 K (s / (K / 4)); rope chunk
  // 4 i + g of row n likewise with swp(n), a base per i.  PV (A = C^T,
  // transposed read): lane s = n of group g reads row 4g + s/4 at channel
  // 16 mb + 4 (s % 4), chunk (2 mb + (s % 4) / 2) ^ swz(row): a base per
  // mb % (K / 2) plus 16 K (mb / (K / 2)).
  constexpr int kGrp = kSwG<NB>, kQkB = kGrp / 4, kPvM = kGrp / 2;
  const int sw_n = swz<NB>(n), sp_n = swp(n);
  uint32_t qk_b[kQkB], pe_b[2];
#pragma unroll
  for (int j = 0; j < kQkB; ++j) qk_b[j] = n * (2 * RP) + 16 * ((4 * j + g) ^ sw_n);
#pragma unroll
  for (int i = 0; i < 2; ++i) pe_b[i] = n * (2 * kP) + 16 * ((4 * i + g) ^ sp_n);
  const int pv_row = 4 * g + (n >> 2);
  const int pv_sw = swz<NB>(pv_row);
  uint32_t pv_m[kPvM];
#pragma unroll
  for (int m = 0; m < kPvM; ++m)
    pv_m[m] = pv_row * (2 * RP) + 16 * ((2 * m + ((n & 3) >> 1)) ^ pv_sw) + 8 * (n & 1);

  // process(k, dry): sub-tile k of this wave.  A dry pass (k = 0) runs the
  // loop body on whatever buffer 0 holds and its results are thrown away: it
  // brings the body into the instruction cache while the first tiles are on
  // their way (a cold first pass costs over a microsecond).
  auto process = [&](int k, bool dry) {
    const int tb = t0 + kSubTok * sub_of(k);
    lds_u8* const sb = wave_lds + (k % NBUF) * G::kSub;
    lds_u8* const pe = sb + G::kLat;
    if constexpr (FUSE) {
      if (fa_wave && k == fa_k && !dry) {
        // The new token replaces the cache row the stream loaded (this wave's
        // own buffer, after its loads landed).
        if constexpr (C_DT == 2) {
#pragma unroll
          for (int i = 0; i < NB; ++i) sb[fa_t * RP + NB * lane + i] = ftok.codes[i];
          if (lane == 0) lds_st<float>(sb + G::kLat + G::kPe + 4 * fa_t, ftok.scale);
        } else {
#pragma unroll
          for (int i = 0; i < NB; ++i) {
            const int ch = NB * lane + i;
            lds_st<uint16_t>(sb + fa_t * (2 * RP) + 16 * ((ch >> 3) ^ swz<NB>(fa_t)) + 2 * (ch & 7), ftok.row[i]);
          }
        }
        if (lane < kP / 2)
          lds_st<uint32_t>(pe + fa_t * (2 * kP) + 16 * ((lane >> 2) ^ swp(fa_t)) + 4 * (lane & 3), ftok.pe);
      }
    }
    float4 scv = make_float4(1.f, 1.f, 1.f, 1.f);
    uint32_t lat = lds_off(sb);
    if constexpr (C_DT == 2) {
      // scales, and the codes decoded into the bf16 staging tile (swizzled as a bf16 tile)
      // Each lane decodes 8 codes (one 16-byte chunk of bf16) per read: the
      // 16 lanes of a store pass then write 16 consecutive chunks of one row,
      // which the swizzle puts on 16 distinct 4-bank groups (with 16 codes
      // per lane, a pass wrote every other chunk of a row: two-way conflicts).
      u32x4v_t sc = ds_read16<0>(lds_off(sb + G::kLat + G::kPe) + 16 * g);
      s16x4_t cv[2 * NB];
      static_for<0, 2 * NB>([&](auto q) { cv[q] = ds_read8<512 * decltype(q)::value>(lds_off(sb) + 8 * lane); });
      lds_fence();
      tie(sc);
      scv = make_float4(u2f(sc.x), u2f(sc.y), u2f(sc.z), u2f(sc.w));
#pragma unroll
      for (int q = 0; q < 2 * NB; ++q) {
        tie(cv[q]);
        const uint2 raw = __builtin_bit_cast(uint2, cv[q]);
        const int o = 512 * q + 8 * lane;
        const int tt = o / RP, c0 = (o % RP) >> 3;  // chunk of the bf16 row
        const uint2 d0 = e4m3x4_to_bf16x4_hw(raw.x), d1 = e4m3x4_to_bf16x4_hw(raw.y);
        lds_st16(stage + tt * (2 * RP) + 16 * (c0 ^ swz<NB>(tt)), make_uint4(d0.x, d0.y, d1.x, d1.y));
      }
      lat = lds_off(stage);
    }
    const uint32_t pe0 = lds_off(pe);

    // operand reads: K (and rope) for S^T, then C^T for the product, whose
    // latency hides under the score and softmax arithmetic
    u32x4v_t kr[2 * NB + 2];
    static_for<0, 2 * NB>([&](auto sI) {
      constexpr int S = decltype(sI)::value;
      kr[S] = ds_read16<16 * kGrp * (S / kQkB)>(lat + qk_b[S % kQkB]);
    });
    kr[2 * NB] = ds_read16<0>(pe0 + pe_b[0]);
    kr[2 * NB + 1] = ds_read16<0>(pe0 + pe_b[1]);
    lds_fence();
#pragma unroll
    for (int i = 0; i < 2 * NB + 2; ++i) tie(kr[i]);
    s16x4_t ctr[4 * NB];
    static_for<0, 4 * NB>([&](auto mI) {
      constexpr int MB = decltype(mI)::value;
      ctr[MB] = ds_read_tr16<16 * kGrp * (MB / kPvM)>(lat + pv_m[MB % kPvM]);
    });

    // S^T = K . Q^T, per head group from the same K registers
    f32x4_t s_c[HG], s_p[HG];
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
      s_c[hg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      s_p[hg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 2 * NB; ++i)
        s_c[hg] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[i]), qb[hg][i], s_c[hg], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const bf16x8_t kp = __builtin_bit_cast(bf16x8_t, kr[2 * NB + i]);
        if constexpr (C_DT == 2) s_p[hg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp, qb[hg][2 * NB + i], s_p[hg], 0, 0, 0);
        else s_c[hg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp, qb[hg][2 * NB + i], s_c[hg], 0, 0, 0);
      }
    }

    const float sc4[4] = {scv.x, scv.y, scv.z, scv.w};
    s16x4_t pb[HG];
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sv = (C_DT == 2) ? (sc4[i] * s_c[hg][i] + s_p[hg][i]) : s_c[hg][i];
        x[i] = tb + 4 * g + i < t1 ? sv * a.scale_log2 : -INFINITY;
      }
      float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      mt = wave_max_rows(mt);  // head n's maximum over the sub-tile (finite: token tb is valid)
      if (__any(mt > m_run[hg] + kLazy)) {
        const float m_new = fmaxf(m_run[hg], mt);
        const float alpha = exp2f(m_run[hg] - m_new);
        m_run[hg] = m_new;
        l_part[hg] *= alpha;
        e_part[hg] *= alpha;
#pragma unroll
        for (int i = 0; i < 4 * NB; ++i) oacc[hg][i] = oacc[hg][i] * alpha;
      }
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = exp2f(x[i] - m_run[hg]);
      // bf16 weights (hardware RNE); l sums exactly those values, so a constant
      // latent row is reproduced exactly; e sums the fp32 weights for the
      // log-sum-exp (the bf16 roundings would move it by up to 2^-9 relative)
      const uint32_t w01 = pack_bf16x2(p[0], p[1]), w23 = pack_bf16x2(p[2], p[3]);
      l_part[hg] += (u2f(w01 << 16) + u2f(w01 & 0xFFFF0000u)) + (u2f(w23 << 16) + u2f(w23 & 0xFFFF0000u));
      e_part[hg] += (p[0] + p[1]) + (p[2] + p[3]);
      uint2 pw = make_uint2(w01, w23);
      if constexpr (C_DT == 2) {
        pw.x = pack_bf16x2(u2f(w01 << 16) * sc4[0], u2f(w01 & 0xFFFF0000u) * sc4[1]);
        pw.y = pack_bf16x2(u2f(w23 << 16) * sc4[2], u2f(w23 & 0xFFFF0000u) * sc4[3]);
      }
      pb[hg] = __builtin_bit_cast(s16x4_t, pw);
    }

    // O^T[16 mb + ., head] += C^T . P^T, per head group from the same C^T registers
    lds_fence();
#pragma unroll
    for (int mb = 0; mb < 4 * NB; ++mb) {
      tie(ctr[mb]);
#pragma unroll
      for (int hg = 0; hg < HG; ++hg)
        oacc[hg][mb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ctr[mb], pb[hg], oacc[hg][mb], 0, 0, 0);
    }
  };

  // The dry pass: the loop body's first run, on buffer 0 while its data (and
  // the query) may still be arriving, with zero queries and the results
  // discarded.  It brings the body into the instruction cache (a cold first
  // pass costs over a microsecond) while the loads are in flight.
#pragma unroll
  for (int hg = 0; hg < HG; ++hg)
#pragma unroll
    for (int i = 0; i < 2 * NB + 2; ++i) qb[hg][i] = as_bf16x8(make_uint4(0u, 0u, 0u, 0u));
  process(0, true);
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
    for (int i = 0; i < 4 * NB; ++i) oacc[hg][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_run[hg] = -INFINITY;
    l_part[hg] = 0.f;
    e_part[hg] = 0.f;
  }

  // Everything issued before the second sub-tile (query, first sub-tile,
  // RoPE row, fused inputs) has landed; the later sub-tiles may still be in
  // flight.
  wait_vm<(G::kFill - 1) * G::kVm>();
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
    for (int s = 0; s < 2 * NB; ++s) vm_release(qraw[hg][s]);
#pragma unroll
    for (int s = 0; s < 2; ++s) vm_release(praw[hg][s]);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    vm_release(cr[s]);
    vm_release(sr[s]);
  }
  if constexpr (FUSE) fused_release(fin);

  // ---- Q^T registers: latent channels >= R zeroed, q_pe rotated (per-op rounded)
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
    for (int s = 0; s < 2 * NB; ++s)
      qb[hg][s] = as_bf16x8(mask_bf16x8(make_uint4(qraw[hg][s][0], qraw[hg][s][1], qraw[hg][s][2], qraw[hg][s][3]),
                                        a.R - (32 * s + 8 * g)));
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      uint32_t wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t cj = (j & 1) ? (cr[s][j >> 1] >> 16) : (cr[s][j >> 1] & 0xFFFF);
        const uint32_t sj = (j & 1) ? (sr[s][j >> 1] >> 16) : (sr[s][j >> 1] & 0xFFFF);
        wv[j] = rope_bf16_packed(bf16_to_f32(praw[hg][s][j] & 0xFFFF), bf16_to_f32(praw[hg][s][j] >> 16),
                                 bf16_to_f32(cj), bf16_to_f32(sj));
      }
      qb[hg][2 * NB + s] = as_bf16x8(make_uint4(wv[0], wv[1], wv[2], wv[3]));
    }
  }

  // The new token's cache row, computed while the first tiles stream in (its
  // inputs were loaded ahead of them).
  if constexpr (FUSE)
    if (fa_wave) {
      ftok = fused_compute<C_DT, NB>(fin, a.fa.eps, a.R, lane,
                                     wave_lds + (G::kLnOwn ? NBUF * G::kSub + G::kStage : (NBUF - 1) * G::kSub));
    }

  for (int k = 0; k < my_n; ++k) {  // uniform
    if (k + G::kCap >= G::kFill && k + G::kCap < my_n) issue(k + G::kCap);
    // sub-tiles issued so far: the fill's kFill (also past my_n), then up to k + kCap
    wait_subtiles<G::kVm, NBUF>(max(G::kFill, min(my_n, k + G::kCap + 1)) - (k + 1));
    process(k, false);
  }
  if constexpr (FUSE)
    if (fa_wave)
      fused_store<C_DT, NB>(a.fa, static_cast<int64_t>(fa_a.b) * a.fa.cache_s + fa_a.pos, ftok, lane);

  // ---- combine the four waves: per head max, sum and O (fixed order)
  // The wave's LDS area is free once its own loads have landed: it stashes
  // its O^T rows and per-head max / l / e there, without waiting for the others.
  wait_vm<0>();  // (the ring's loads past the wave's own sub-tiles included)
  // (stash_of(v, hg): wave v's stash of head group hg)
  auto stash_of = [&](int v, int hg) {
    return reinterpret_cast<float*>(lds_raw + v * G::kWave) + hg * G::kStashG;
  };
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
    float l_w = l_part[hg] + shfl_xor_f32(l_part[hg], 16);
    l_w += shfl_xor_f32(l_w, 32);
    float e_w = e_part[hg] + shfl_xor_f32(e_part[hg], 16);
    e_w += shfl_xor_f32(e_w, 32);
    float* const mine = stash_of(w, hg);
    if (g == 0) {
      mine[kH * G::kCombRow + n] = m_run[hg];
      mine[kH * G::kCombRow + kH + n] = l_w;
      mine[kH * G::kCombRow + 2 * kH + n] = e_w;
    }
    // lane (n, g) holds O^T[16 mb + 4 g + i][head n]
#pragma unroll
    for (int mb = 0; mb < 4 * NB; ++mb)
      *reinterpret_cast<float4*>(mine + n * G::kCombRow + 16 * mb + 4 * g) =
          make_float4(oacc[hg][mb][0], oacc[hg][mb][1], oacc[hg][mb][2], oacc[hg][mb][3]);
  }
  __syncthreads();  // every wave's stash is written

  // wave w finishes heads 4w .. 4w + 3 of each head group: lane -> head
  // 4w + g, channels 64 i + 4 n .. +4 for i < NB (the 16 lanes of a head
  // read and write consecutive 16-byte pieces); hh is the head in the launch
  const int h = kDecWaves * w + g, c0 = 4 * n;
#pragma unroll 1
  for (int hg = 0; hg < HG; ++hg) {
    const int hh = kH * hg + h;
    float mw[kDecWaves], lw[kDecWaves], ew[kDecWaves];
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < kDecWaves; ++v) {
      const float* ml = stash_of(v, hg) + kH * G::kCombRow;
      mw[v] = ml[h];
      lw[v] = ml[kH + h];
      ew[v] = ml[2 * kH + h];
      M = fmaxf(M, mw[v]);
    }
    float sc[kDecWaves], Ltot = 0.f, Etot = 0.f;
#pragma unroll
    for (int v = 0; v < kDecWaves; ++v) {
      sc[v] = mw[v] == -INFINITY ? 0.f : exp2f(mw[v] - M);
      Ltot += sc[v] * lw[v];
      Etot += sc[v] * ew[v];
    }
    const float inv = Ltot > 0.f ? 1.f / Ltot : 0.f;
    float o[4 * NB];
#pragma unroll
    for (int i = 0; i < 4 * NB; ++i) o[i] = 0.f;
#pragma unroll
    for (int v = 0; v < kDecWaves; ++v) {
      const float* src = stash_of(v, hg) + h * G::kCombRow + c0;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const float4 t = *reinterpret_cast<const float4*>(src + 64 * i);
        o[4 * i + 0] += sc[v] * t.x;
        o[4 * i + 1] += sc[v] * t.y;
        o[4 * i + 2] += sc[v] * t.z;
        o[4 * i + 3] += sc[v] * t.w;
      }
    }
    const float lse2 = Etot > 0.f ? M + __log2f(Etot) : -INFINITY;  // log2 domain
    if (ns <= 1) {
      uint16_t* op = static_cast<uint16_t*>(a.o_lat) + r * a.o_rs + hh * a.o_hs + c0;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        uint2 pk;
        pk.x = pack_bf16x2(o[4 * i] * inv, o[4 * i + 1] * inv);
        pk.y = pack_bf16x2(o[4 * i + 2] * inv, o[4 * i + 3] * inv);
        *reinterpret_cast<uint2*>(op + 64 * i) = pk;
      }
      if (a.lse_out && n == 0) a.lse_out[static_cast<int64_t>(r) * HT + hh] = lse2 * kLn2;
      continue;
    }
    // partials: non-temporal stores (every workgroup writes at its end, and the
    // merge reads them in the next launch, from another XCD's view of memory)
    const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * HT + hh;
    float* op = a.o_part + pidx * RP + c0;
#pragma unroll
    for (int i = 0; i < NB; ++i)
      __builtin_nontemporal_store(f32x4_t{o[4 * i] * inv, o[4 * i + 1] * inv, o[4 * i + 2] * inv, o[4 * i + 3] * inv},
                                  reinterpret_cast<f32x4_t*>(op + 64 * i));
    if (n == 0) __builtin_nontemporal_store(lse2 * kLn2, a.lse_part + pidx);
  }
}

// ===========================================================================
// Ranks above 512 (R_pad = 64 NB, NB = 9 .. 16), bf16 model and cache.
// ===========================================================================
// The per-wave design above keeps a wave's O^T for all R_pad channels (4 NB
// accumulators) and Q^T for R_pad + 64 in registers; past NB = 8 that no
// longer fits.  Here the four waves of a workgroup share every sub-tile of
// the split and divide the channels instead: wave w owns the 64-channel
// blocks c = w, w + 4, w + 8, w + 12 (those below NB) and rope dimensions
// 16 w .. 16 w + 15.  Per 16-token sub-tile a wave
//   * streams its own channel blocks of the 16 latent rows (2 KB each, laid
//     out as a one-block sub-tile of the kernel above, with the same 8-chunk
//     swizzle) and its 32-byte slice of the 16 rope rows into its own LDS
//     ring with global_load_lds_dwordx4; a wave with fewer blocks than the
//     most loaded one re-reads its last block into the spare slot, so every
//     wave issues kVm instructions per sub-tile and the waits stay fixed;
//   * forms its partial S^T[16 tok x 16 heads] over its channels
//     (mfma_f32_16x16x32_bf16) and rope slice (mfma_f32_16x16x16_bf16);
//   * writes the partial to a double-buffered LDS exchange area, passes one
//     barrier, and reads the four partials back, added in wave order, so
//     every wave holds the same scores and runs the same online softmax;
//   * accumulates O^T for its own channels (C^T read transposed from LDS).
// Each wave then writes its own channels of o_lat or of the split's partial;
// wave 0 writes the log-sum-exp.  Numerics are the kernel's above: bf16
// weights in the product, o normalised by their sum, the LSE from the fp32
// weights, per-op rounded q_pe RoPE, query channels >= R zeroed.
namespace {
template <int C_DT, int NB>
struct WideGeo {
  static constexpr int RP = 64 * NB;
  static constexpr int NBW = (NB + kDecWaves - 1) / kDecWaves;  // channel blocks of the most loaded wave
  static constexpr int kBlk = kSubTok * 128;                    // one 64-channel block of 16 bf16 rows
  static constexpr int kBlkC = C_DT == 2 ? kSubTok * 64 : kBlk;  // ring bytes of a block (e4m3: codes)
  static constexpr int kPe = 1024;                              // 16 rope slices of 32 B (+ 512 B re-read)
  static constexpr int kSc = C_DT == 2 ? 256 : 0;               // e4m3: 4 copies of the 16 scales
  static constexpr int kSub = NBW * kBlkC + kPe + kSc;          // a wave's ring bytes of one sub-tile
  static constexpr int kVm = (C_DT == 2 ? NBW + 2 : 2 * NBW + 1);  // DMA instructions per sub-tile
  static constexpr int kStage = C_DT == 2 ? NBW * kBlk : 0;     // e4m3: the wave's blocks decoded to bf16
  static constexpr int NBUF = 3, kFill = 2, kCap = 2;
  static constexpr int kXch = 2 * kDecWaves * 1024;             // two exchange buffers of 4 waves x 64 lanes x 16 B
  static constexpr int kWave = NBUF * kSub + kStage;
  static constexpr int kLds = kDecWaves * kWave + kXch;
  static_assert(kLds <= kLdsMax, "LDS budget");
  static_assert((kFill + 1) * kVm < 64, "vmcnt range");
};

__device__ __forceinline__ void ds_write16(uint32_t addr, f32x4_t v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
}  // namespace

template <int C_DT, int NB>
__global__ __launch_bounds__(kDecWaves * 64, 1) void mla_decode_wide(DecodeArgs a) {
  using G = WideGeo<C_DT, NB>;
  constexpr int RP = G::RP, NBW = G::NBW, NBUF = G::NBUF;
  __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[G::kLds];
  lds_u8* const lds = (lds_u8*)(lds_raw);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;

  // ---- workgroup -> (row, split), as in mla_decode_dma
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
    ra = bs.addr;
  } else {
    ra = row_addr(a.ad, r);
  }

  // ---- this wave's query: latent blocks c = w + 4 i (lane: head n, channels
  // 64 c + 32 s + 8 g .. + 8), rope dims 16 w + 4 g .. + 4
  uint32_t qraw[NBW][2][4], praw[2];
  const uint16_t* qa = static_cast<const uint16_t*>(a.q_abs) + r * a.qa_rs + n * a.qa_hs;
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int c = min(w + kDecWaves * i, NB - 1);  // a spare block re-reads a valid one (never used)
#pragma unroll
    for (int s = 0; s < 2; ++s) vm_load<4>(qa + 64 * c + 32 * s + 8 * g, qraw[i][s]);
  }
  vm_load<2>(static_cast<const uint16_t*>(a.q_pe) + r * a.qp_rs + n * a.qp_hs + 16 * w + 4 * g, praw);
  int rp = ra.rope;
  rp = rp < 0 ? 0 : (rp >= a.rope_len ? static_cast<int>(a.rope_len) - 1 : rp);
  uint32_t crw[1], srw[1];
  vm_load<1>(static_cast<const uint16_t*>(a.cos_tab) + static_cast<int64_t>(rp) * (kP / 2) + 8 * w + 2 * g, crw);
  vm_load<1>(static_cast<const uint16_t*>(a.sin_tab) + static_cast<int64_t>(rp) * (kP / 2) + 8 * w + 2 * g, srw);

  const int b = ra.b;
  int L = ra.pos;
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const RowSplits rsp = row_splits(L, a.n_splits, a.min_chunk, bal_chunk);
  const int ns = rsp.ns;
  if (split >= ns && !(ns == 0 && split == 0)) {
    wait_vm<0>();
    return;
  }
  if (a.balance <= 0 && ns > 0) split = ns - 1 - split;
  const int t0 = split * rsp.chunk;  // a multiple of 16
  const int t1 = min(L, t0 + rsp.chunk);
  const int t_last = t1 > 0 ? t1 - 1 : 0;
  const int n_sub = t1 > t0 ? (t1 - t0 + kSubTok - 1) / kSubTok : 0;
  const int64_t row0 = static_cast<int64_t>((b < 0 || b >= a.cache_b) ? 0 : b) * a.cache_s;

  // ---- the wave's ring: per sub-tile NBW latent blocks, then the rope slices
  lds_u8* const wave_lds = lds + w * G::kWave;
  lds_u8* const xch = lds + kDecWaves * G::kWave;
  const uint8_t* const ckv = static_cast<const uint8_t*>(a.ckv);
  const uint8_t* const kpe = static_cast<const uint8_t*>(a.kpe);
  // DMA lane offsets: latent instruction q of a block covers rows 8 q + lane / 8,
  // slot lane % 8 holding chunk (lane % 8) ^ swz<1>(row); rope: row (lane / 2) % 16,
  // half lane % 2 of the wave's 32 bytes (lanes 32 .. 63 re-read lanes 0 .. 31's)
  int lat_row[2];
  uint32_t lat_col[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    lat_row[q] = 8 * q + (lane >> 3);
    lat_col[q] = 16 * ((lane & 7) ^ swz<1>(lat_row[q]));
  }
  const int pe_row = (lane >> 1) & 15;
  const uint32_t pe_col = 32 * w + 16 * (lane & 1);
  auto issue = [&](int k) {
    const int tb = t0 + kSubTok * k;
    lds_u8* const dst = wave_lds + (k % NBUF) * G::kSub;
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int c = min(w + kDecWaves * i, NB - 1);
      if constexpr (C_DT == 2) {
        // e4m3 codes as they lie: row lane / 4, bytes 16 (lane % 4) of the block's 64
        const int tok = min(tb + (lane >> 2), t_last);
        dma16(ckv + (row0 + tok) * RP + 64 * c + 16 * (lane & 3), dst + i * G::kBlkC);
      } else {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int tok = min(tb + lat_row[q], t_last);
          dma16(ckv + (row0 + tok) * (2 * RP) + 128 * c + lat_col[q], dst + i * G::kBlk + 1024 * q);
        }
      }
    }
    const int tok = min(tb + pe_row, t_last);
    dma16(kpe + (row0 + tok) * (2 * kP) + pe_col, dst + NBW * G::kBlkC);
    if constexpr (C_DT == 2) dma4(a.ckv_scale + row0 + min(tb + (lane & 15), t_last), dst + NBW * G::kBlkC + G::kPe);
  };
  issue(0);
#pragma unroll
  for (int k = 1; k < G::kFill; ++k) issue(k);  // past n_sub: re-reads the split's last row

  // operand addresses within one block (the one-block layout of mla_decode_dma)
  const int sw_n = swz<1>(n);
  uint32_t qk_b[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) qk_b[s] = n * 128 + 16 * ((4 * s + g) ^ sw_n);
  const int pv_row = 4 * g + (n >> 2);
  const int pv_sw = swz<1>(pv_row);
  uint32_t pv_m[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) pv_m[m] = pv_row * 128 + 16 * ((2 * m + ((n & 3) >> 1)) ^ pv_sw) + 8 * (n & 1);
  const uint32_t pe_rd = NBW * G::kBlkC + n * 32 + 8 * g;
  lds_u8* const stage_p = wave_lds + NBUF * G::kSub;  // e4m3 only
  const uint32_t stage = lds_off(stage_p);
  const uint32_t xw = lds_off(xch) + 1024 * w + 16 * lane;  // this wave's exchange slot (buffer 0)
  const uint32_t xr = lds_off(xch) + 16 * lane;             // wave v's slot: + 1024 v

  f32x4_t oacc[4 * NBW];
#pragma unroll
  for (int i = 0; i < 4 * NBW; ++i) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f, e_part = 0.f;

  // queries (and everything else issued before the DMAs) have landed
  wait_vm<G::kFill * G::kVm>();
#pragma unroll
  for (int i = 0; i < NBW; ++i)
#pragma unroll
    for (int s = 0; s < 2; ++s) vm_release(qraw[i][s]);
  vm_release(praw);
  vm_release(crw);
  vm_release(srw);
  bf16x8_t qb[NBW][2];
#pragma unroll
  for (int i = 0; i < NBW; ++i)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c = w + kDecWaves * i;
      qb[i][s] = as_bf16x8(mask_bf16x8(make_uint4(qraw[i][s][0], qraw[i][s][1], qraw[i][s][2], qraw[i][s][3]),
                                       a.R - (64 * c + 32 * s + 8 * g)));
    }
  uint32_t qp[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t cj = j ? (crw[0] >> 16) : (crw[0] & 0xFFFF);
    const uint32_t sj = j ? (srw[0] >> 16) : (srw[0] & 0xFFFF);
    qp[j] = rope_bf16_packed(bf16_to_f32(praw[j] & 0xFFFF), bf16_to_f32(praw[j] >> 16), bf16_to_f32(cj),
                             bf16_to_f32(sj));
  }
  const s16x4_t qpe = __builtin_bit_cast(s16x4_t, make_uint2(qp[0], qp[1]));

  for (int k = 0; k < n_sub; ++k) {  // uniform
    if (k + G::kCap >= G::kFill && k + G::kCap < n_sub) issue(k + G::kCap);
    wait_subtiles<G::kVm, NBUF>(max(G::kFill, min(n_sub, k + G::kCap + 1)) - (k + 1));
    const int tb = t0 + kSubTok * k;
    const uint32_t sb = lds_off(wave_lds + (k % NBUF) * G::kSub);
    uint32_t lat = sb;  // the bf16 blocks the operand reads take
    float4 scv = make_float4(1.f, 1.f, 1.f, 1.f);
    if constexpr (C_DT == 2) {
      // scales of the lane's tokens 4 g .. 4 g + 3, and the codes decoded into
      // the staging tile in the bf16 ring layout (each lane: 8 codes -> one
      // 16-byte chunk, two chunks per block)
      u32x4v_t sc = ds_read16<0>(sb + NBW * G::kBlkC + G::kPe + 16 * g);
      s16x4_t cv[NBW][2];
      static_for<0, NBW>([&](auto iI) {
        constexpr int I = decltype(iI)::value;
        cv[I][0] = ds_read8<I * G::kBlkC>(sb + 8 * lane);
        cv[I][1] = ds_read8<I * G::kBlkC + 512>(sb + 8 * lane);
      });
      lds_fence();
      tie(sc);
      scv = make_float4(u2f(sc.x), u2f(sc.y), u2f(sc.z), u2f(sc.w));
#pragma unroll
      for (int i = 0; i < NBW; ++i)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          tie(cv[i][q]);
          const uint2 raw = __builtin_bit_cast(uint2, cv[i][q]);
          const int o = 512 * q + 8 * lane;  // code offset in the block: row o / 64, chunk (o % 64) / 8
          const int tt = o >> 6, c0 = (o & 63) >> 3;
          const uint2 d0 = e4m3x4_to_bf16x4_hw(raw.x), d1 = e4m3x4_to_bf16x4_hw(raw.y);
          lds_st16(stage_p + i * G::kBlk + tt * 128 + 16 * (c0 ^ swz<1>(tt)), make_uint4(d0.x, d0.y, d1.x, d1.y));
        }
      lat = stage;
    }
    u32x4v_t kr[NBW][2];
    static_for<0, NBW>([&](auto iI) {
      constexpr int I = decltype(iI)::value;
      kr[I][0] = ds_read16<I * G::kBlk>(lat + qk_b[0]);
      kr[I][1] = ds_read16<I * G::kBlk>(lat + qk_b[1]);
    });
    s16x4_t kp = ds_read8<0>(sb + pe_rd);
    lds_fence();
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      tie(kr[i][0]);
      tie(kr[i][1]);
    }
    tie(kp);
    s16x4_t ctr[NBW][4];
    static_for<0, NBW>([&](auto iI) {
      constexpr int I = decltype(iI)::value;
      static_for<0, 4>([&](auto mI) {
        constexpr int M = decltype(mI)::value;
        ctr[I][M] = ds_read_tr16<I * G::kBlk>(lat + pv_m[M]);
      });
    });

    // this wave's partial scores, then the exchange
    f32x4_t sp = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NBW; ++i)
      if (w + kDecWaves * i < NB) {  // uniform
        sp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[i][0]), qb[i][0], sp, 0, 0, 0);
        sp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[i][1]), qb[i][1], sp, 0, 0, 0);
      }
    // The rope term has an accumulator of its own, added on the VALU: an
    // mfma_f32_16x16x16 taking the 16x16x32 chain's result as its C operand
    // got too few wait states on gfx950 and read the accumulator before the
    // chain's last product had landed (the last channel block's scores were
    // lost); the VALU adds also keep the inline-asm store below off a
    // matrix-core result.
    const f32x4_t spe = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(kp, qpe, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    // (e4m3: the token's scale multiplies the latent part, as in mla_decode_dma)
    const f32x4_t stot = f32x4_t{scv.x * sp[0] + spe[0], scv.y * sp[1] + spe[1], scv.z * sp[2] + spe[2],
                                 scv.w * sp[3] + spe[3]};
    const uint32_t xo = 4096 * (k & 1);
    ds_write16(xw + xo, stot);
    lds_fence();  // the partial (and the C^T reads) are in LDS
    __builtin_amdgcn_s_barrier();
    u32x4v_t xv[kDecWaves];
    static_for<0, kDecWaves>([&](auto vI) {
      constexpr int V = decltype(vI)::value;
      xv[V] = ds_read16<1024 * V>(xr + xo);
    });
    lds_fence();
#pragma unroll
    for (int v = 0; v < kDecWaves; ++v) tie(xv[v]);
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sv = ((u2f(xv[0][i]) + u2f(xv[1][i])) + u2f(xv[2][i])) + u2f(xv[3][i]);
      x[i] = tb + 4 * g + i < t1 ? sv * a.scale_log2 : -INFINITY;
    }
    float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mt = wave_max_rows(mt);  // head n's maximum over the sub-tile (finite: token tb is valid)
    if (__any(mt > m_run + kLazy)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      l_part *= alpha;
      e_part *= alpha;
#pragma unroll
      for (int i = 0; i < 4 * NBW; ++i) oacc[i] = oacc[i] * alpha;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = exp2f(x[i] - m_run);
    const uint32_t w01 = pack_bf16x2(p[0], p[1]), w23 = pack_bf16x2(p[2], p[3]);
    l_part += (u2f(w01 << 16) + u2f(w01 & 0xFFFF0000u)) + (u2f(w23 << 16) + u2f(w23 & 0xFFFF0000u));
    e_part += (p[0] + p[1]) + (p[2] + p[3]);
    uint2 pw = make_uint2(w01, w23);
    if constexpr (C_DT == 2) {
      pw.x = pack_bf16x2(u2f(w01 << 16) * scv.x, u2f(w01 & 0xFFFF0000u) * scv.y);
      pw.y = pack_bf16x2(u2f(w23 << 16) * scv.z, u2f(w23 & 0xFFFF0000u) * scv.w);
    }
    const s16x4_t pb = __builtin_bit_cast(s16x4_t, pw);
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
#pragma unroll
      for (int m = 0; m < 4; ++m) tie(ctr[i][m]);
      if (w + kDecWaves * i < NB)  // uniform
#pragma unroll
        for (int m = 0; m < 4; ++m)
          oacc[4 * i + m] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ctr[i][m], pb, oacc[4 * i + m], 0, 0, 0);
    }
  }
  wait_vm<0>();  // the ring's loads past the split's sub-tiles

  // ---- the wave's channels of head n: lane (n, g) holds O^T[16 m + 4 g + j][n]
  // of each block; l and e summed over the head's four lane groups
  float l_w = l_part + shfl_xor_f32(l_part, 16);
  l_w += shfl_xor_f32(l_w, 32);
  float e_w = e_part + shfl_xor_f32(e_part, 16);
  e_w += shfl_xor_f32(e_w, 32);
  const float inv = l_w > 0.f ? 1.f / l_w : 0.f;
  const float lse2 = e_w > 0.f ? m_run + __log2f(e_w) : -INFINITY;  // log2 domain
  if (ns <= 1) {
    uint16_t* op = static_cast<uint16_t*>(a.o_lat) + r * a.o_rs + n * a.o_hs + 4 * g;
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int c = w + kDecWaves * i;
      if (c < NB)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          uint2 pk;
          pk.x = pack_bf16x2(oacc[4 * i + m][0] * inv, oacc[4 * i + m][1] * inv);
          pk.y = pack_bf16x2(oacc[4 * i + m][2] * inv, oacc[4 * i + m][3] * inv);
          *reinterpret_cast<uint2*>(op + 64 * c + 16 * m) = pk;
        }
    }
    if (a.lse_out && w == 0 && g == 0) a.lse_out[static_cast<int64_t>(r) * kH + n] = lse2 * kLn2;
    return;
  }
  const int64_t pidx = (static_cast<int64_t>(r) * a.n_splits + split) * kH + n;
  float* op = a.o_part + pidx * RP + 4 * g;
#pragma unroll
  for (int i = 0; i < NBW; ++i) {
    const int c = w + kDecWaves * i;
    if (c < NB)
#pragma unroll
      for (int m = 0; m < 4; ++m)
        __builtin_nontemporal_store(f32x4_t{oacc[4 * i + m][0] * inv, oacc[4 * i + m][1] * inv,
                                            oacc[4 * i + m][2] * inv, oacc[4 * i + m][3] * inv},
                                    reinterpret_cast<f32x4_t*>(op + 64 * c + 16 * m));
  }
  if (w == 0 && g == 0) __builtin_nontemporal_store(lse2 * kLn2, a.lse_part + pidx);
}

// ===========================================================================
// Measurement kernels (no reference counterpart; used by bench.py's ceiling
// legs, never by the module).
// ===========================================================================
// mla_stream_probe: a decode launch's cache stream alone.  The same grid,
// workgroup shape, LDS ring, split plan (static), sub-tile deal, DMA
// instructions and count-based waits as mla_decode_dma, with no query loads,
// no arithmetic and no epilogue.  Each wave folds one 16-byte word of every
// sub-tile it receives into a checksum stored at sink[workgroup * 256 +
// thread], so the stream is observable.  Its duration is the floor of any
// decode launch with this access pattern on this GPU.
template <int C_DT, int NB>
__global__ __launch_bounds__(kDecWaves * 64, 1) void mla_stream_probe(DecodeArgs a, uint32_t* sink) {
  using G = DecGeo<C_DT, NB>;
  constexpr int NBUF = G::NBUF;
  __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[G::kLds];
  lds_u8* const lds = (lds_u8*)(lds_raw);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.y;
  const TokAddr ra = row_addr(a.ad, r);
  const int b = ra.b;
  int L = ra.pos;
  if (L > a.cache_s) L = static_cast<int>(a.cache_s);
  if (b < 0 || b >= a.cache_b) L = 0;
  const RowSplits rsp = row_splits(L, a.n_splits, a.min_chunk, 0);
  uint32_t acc = 0;
  if (static_cast<int>(blockIdx.x) < rsp.ns) {  // uniform
    const int split = rsp.ns - 1 - static_cast<int>(blockIdx.x);
    const int t0 = split * rsp.chunk;
    const int t1 = min(L, t0 + rsp.chunk);
    const int64_t row0 = static_cast<int64_t>(b) * a.cache_s;
    lds_u8* const wave_lds = lds + w * G::kWave;
    const SubStream<C_DT, NB, 1> ss(t0, t1, w, lane, row0, a.ckv, a.kpe, a.ckv_scale, wave_lds);
#pragma unroll
    for (int k = 0; k < G::kFill; ++k) ss.issue(k, lane);
    for (int k = 0; k < ss.my_n; ++k) {  // uniform
      if (k + G::kCap >= G::kFill && k + G::kCap < ss.my_n) ss.issue(k + G::kCap, lane);
      wait_subtiles<G::kVm, NBUF>(max(G::kFill, min(ss.my_n, k + G::kCap + 1)) - (k + 1));
      u32x4v_t v = ds_read16<0>(lds_off(wave_lds + (k % NBUF) * G::kSub) + 16 * lane);
      lds_fence();
      tie(v);
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    wait_vm<0>();
  }
  sink[(static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * (kDecWaves * 64) + threadIdx.x] = acc;
}

// ===========================================================================
// Launchers behind the C-ABI (argument validation lives in mla_abi.cpp).
// ===========================================================================
namespace {
// The instance for (cache dtype, fused append, head groups): two head groups
// (32 heads) are built for R_pad <= 256, where both groups' queries and
// accumulators fit one wave's registers.
template <int NB>
const void* decode_kernel(int c_dt, bool fuse, int hg) {
  if (hg == 2) {
    if constexpr (NB <= 4) {
      if (c_dt == 1 && !fuse) return reinterpret_cast<const void*>(&mla_decode_dma<1, false, NB, 2>);
      if (c_dt == 2 && !fuse) return reinterpret_cast<const void*>(&mla_decode_dma<2, false, NB, 2>);
      if (c_dt == 1) return reinterpret_cast<const void*>(&mla_decode_dma<1, true, NB, 2>);
      if (c_dt == 2) return reinterpret_cast<const void*>(&mla_decode_dma<2, true, NB, 2>);
    }
    return nullptr;
  }
  if (hg != 1) return nullptr;
  if (c_dt == 1 && !fuse) return reinterpret_cast<const void*>(&mla_decode_dma<1, false, NB, 1>);
  if (c_dt == 2 && !fuse) return reinterpret_cast<const void*>(&mla_decode_dma<2, false, NB, 1>);
  if (c_dt == 1) return reinterpret_cast<const void*>(&mla_decode_dma<1, true, NB, 1>);
  if (c_dt == 2) return reinterpret_cast<const void*>(&mla_decode_dma<2, true, NB, 1>);
  return nullptr;
}
}  // namespace

int launch_decode(const DecodeArgs& a, int dt, int c_dt, hipStream_t s) {
  if (a.n_rows == 0) return 0;
  if (dt == 1 && (c_dt == 1 || c_dt == 2) && padded_rank(a.R) > 64 * kMaxNB) {
    // bf16 models above rank 512: the channel-split MFMA kernel (no fused append, 16 heads)
    if (a.fa.kv_in != nullptr || a.H != kH) return -1;
    const dim3 grid = a.balance > 0 ? dim3(a.balance, 1) : dim3(a.n_splits, a.n_rows);
    const int rc = with_nb_wide(a.R, [&](auto nb) {
      constexpr int NB = decltype(nb)::value;
      if constexpr (NB <= kMaxNB) {
        return -1;
      } else {
        void* args[] = {const_cast<DecodeArgs*>(&a)};
        const void* fn = c_dt == 2 ? reinterpret_cast<const void*>(&mla_decode_wide<2, NB>)
                                   : reinterpret_cast<const void*>(&mla_decode_wide<1, NB>);
        return hipLaunchKernel(fn, grid, dim3(kDecWaves * 64), args, 0, s) == hipSuccess
                   ? 0
                   : -2;
      }
    });
    if (rc != 0) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -2;
  }
  if (dt == 0 || padded_rank(a.R) > 64 * kMaxNB) {
    // the VALU kernel: fp32 models
    if (a.fa.kv_in != nullptr || a.H != kH) return -1;
    return launch_decode_vec(a, dt, c_dt, s);
  }
  if (dt != 1 || a.H % kH != 0) return -1;
  const int hg = a.H / kH;
  const dim3 grid = a.balance > 0 ? dim3(a.balance, 1) : dim3(a.n_splits, a.n_rows);
  const bool fuse = a.fa.kv_in != nullptr;
  const int rc = with_nb(a.R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    const void* fn = decode_kernel<NB>(c_dt, fuse, hg);
    if (!fn) return -1;
    void* args[] = {const_cast<DecodeArgs*>(&a)};
    return hipLaunchKernel(fn, grid, dim3(kDecWaves * 64), args, 0, s) == hipSuccess ? 0 : -2;
  });
  if (rc != 0) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// The stream probe over a decode launch's rows (bf16 model; static plan).
int launch_stream_probe(const DecodeArgs& a, int c_dt, uint32_t* sink, hipStream_t s) {
  if (a.n_rows == 0) return 0;
  if (a.balance > 0 || (c_dt != 1 && c_dt != 2)) return -1;
  const int rc = with_nb(a.R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    const void* fn = c_dt == 1 ? reinterpret_cast<const void*>(&mla_stream_probe<1, NB>)
                               : reinterpret_cast<const void*>(&mla_stream_probe<2, NB>);
    void* args[] = {const_cast<DecodeArgs*>(&a), &sink};
    return hipLaunchKernel(fn, dim3(a.n_splits, a.n_rows), dim3(kDecWaves * 64), args, 0, s) == hipSuccess ? 0 : -2;
  });
  if (rc != 0) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Workgroups of a decode launch one CU holds at once: the MFMA kernel takes a
// whole CU (its LDS ring), the fp32 kernel's own count.
int decode_blocks_per_cu(int dt, int c_dt, int R, bool fuse, int* blocks) {
  if (dt == 1 && (c_dt == 1 || c_dt == 2) && padded_rank(R) > 64 * kMaxNB) {
    if (fuse) return -1;
    *blocks = 1;  // the wide kernel's ring takes a CU
    return 0;
  }
  if (dt == 0 || padded_rank(R) > 64 * kMaxNB) return fuse ? -1 : decode_vec_blocks_per_cu(dt, c_dt, R, blocks);
  if (dt != 1) return -1;
  return with_nb(R, [&](auto nb) {
    constexpr int NB = decltype(nb)::value;
    const void* fn = decode_kernel<NB>(c_dt, fuse, 1);
    if (!fn) return -1;
    int nblk = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nblk, fn, kDecWaves * 64, 0) != hipSuccess || nblk < 1)
      return -2;
    *blocks = 1;
    return 0;
  });
}

}  // namespace swamla
