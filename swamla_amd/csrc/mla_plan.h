// mla_plan.h — split plan and token / row addressing shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "mla_args.h"
#include "numerics.h"

namespace swamla {

// ---------------------------------------------------------------------------
// Split plan (shared by decode and merge; mirrored by mla_split_count).
// ---------------------------------------------------------------------------
SW_HD int split_chunk(int L, int n_splits, int min_chunk) {
  int c = (L + n_splits - 1) / n_splits;
  if (c < min_chunk) c = min_chunk;
  return (c + 15) & ~15;
}
SW_HD int split_count(int L, int n_splits, int min_chunk) {
  if (L <= 0) return 0;
  int c = split_chunk(L, n_splits, min_chunk);
  return (L + c - 1) / c;
}

// ---------------------------------------------------------------------------
// Length-balanced split plan (ragged batches).  One chunk length c, a multiple
// of 64 tokens, for the whole launch, chosen from all rows' lengths: the
// smallest c >= min_chunk with ceil(L_r / c) <= n_splits for every row and
// sum_r max(1, ceil(L_r / c)) <= target (an empty row still takes one
// workgroup, which writes its zero output).  Row r then takes
// ceil(L_r / c) workgroups and is cut into that many near-equal splits
// (row_splits).  A solution exists whenever n_rows <= target.  The counts
// are kept in 64-token tiles: ceil(L / 64c') = ceil(ceil(L / 64) / c').
// Balanced plans cover caches of at most 2^24 positions, so tile counts and
// their sums stay below 2^26.
// ---------------------------------------------------------------------------
constexpr int kBalanceMaxRows = 256;
constexpr int64_t kBalanceMaxSeq = int64_t(1) << 24;

SW_HD int ceil_div_pos(int a, int b) { return (a + b - 1) / b; }

// ceil(a / b) for 0 <= a < 2^20, 1 <= b < 2^20 from the fp32 reciprocal: a and
// b are exact in fp32 and the product is within 1/4 of a / b, so one
// correction of the truncated quotient gives floor(a / b).
__device__ __forceinline__ int ceil_div_small(int a, int b) {
  int q = static_cast<int>(static_cast<float>(a) * __builtin_amdgcn_rcpf(static_cast<float>(b)));
  int rem = a - q * b;
  if (rem < 0) {
    --q;
    rem += b;
  } else if (rem >= b) {
    ++q;
    rem -= b;
  }
  return q + (rem > 0 ? 1 : 0);
}

// Search bounds in tiles: lo = the smallest chunk the constraints allow,
// hi = a chunk known to satisfy them (sum ceil(lt / hi) <= sum lt / hi +
// n_rows <= target, or every row in one piece).
SW_HD void balanced_bounds(int sum_tiles, int max_tiles, int n_rows, int n_splits, int min_chunk, int target,
                           int* lo, int* hi) {
  int l = ceil_div_pos(min_chunk > 0 ? min_chunk : 1, 64);
  const int l2 = ceil_div_pos(max_tiles, n_splits), l3 = ceil_div_pos(sum_tiles, target);
  l = l2 > l ? l2 : l;
  l = l3 > l ? l3 : l;
  int h = target > n_rows ? ceil_div_pos(sum_tiles, target - n_rows) : max_tiles;
  h = h < max_tiles ? h : max_tiles;
  *lo = l;
  *hi = h > l ? h : l;
}

// Splits of a row of L tokens.  Static plan (bal_chunk == 0): split_count /
// split_chunk.  Balanced plan with chunk c: the row keeps its
// ceil(ceil(L / 64) / (c / 64)) workgroups of the plan and is cut into
// near-equal pieces, split_count / split_chunk with that many splits and no
// minimum (a piece of a row never exceeds c).
struct RowSplits {
  int ns, chunk;
};
SW_HD RowSplits row_splits(int L, int n_splits, int min_chunk, int bal_chunk) {
  if (bal_chunk > 0) {
    const int lt = L > 0 ? (L >> 6) + ((L & 63) != 0) : 0;
    n_splits = lt > 0 ? ceil_div_pos(lt, bal_chunk >> 6) : 1;  // < 2^18
    min_chunk = 1;
  }
  const int ns = split_count(L, n_splits, min_chunk);
  return {ns, ns ? split_chunk(L, n_splits, min_chunk) : 0};
}

// Host restatement over already clamped lengths (exported as
// mla_balanced_chunk; each length <= kBalanceMaxSeq).  Returns c in tokens.
inline int balanced_chunk_host(const int32_t* lens, int n_rows, int n_splits, int min_chunk, int target) {
  int sum = 0;
  int mx = 0;
  for (int r = 0; r < n_rows; ++r) {
    const int lt = lens[r] > 0 ? (lens[r] >> 6) + ((lens[r] & 63) != 0) : 0;
    sum += lt;
    mx = lt > mx ? lt : mx;
  }
  auto blocks = [&](int ct) {
    int n = 0;
    for (int r = 0; r < n_rows; ++r) n += lens[r] > 0 ? ceil_div_pos((lens[r] >> 6) + ((lens[r] & 63) != 0), ct) : 1;
    return n;
  };
  int lo, hi;
  balanced_bounds(sum, mx, n_rows, n_splits, min_chunk, target, &lo, &hi);
  while (lo < hi) {
    const int mid = lo + (hi - lo) / 2;
    if (blocks(mid) <= target) hi = mid;
    else lo = mid + 1;
  }
  return 64 * lo;
}

// ---------------------------------------------------------------------------
// Addressing of tokens (append) and query rows (decode / merge).
// ---------------------------------------------------------------------------
struct TokAddr {
  int b, pos, rope;
};

// Append: cache row, destination position, RoPE table row of token i.
__device__ __forceinline__ TokAddr tok_addr(const Addressing& ad, int i) {
  if (ad.start_pos) {
    const int b = i / ad.T, t = i - b * ad.T;
    const int p = ad.start_pos[b] + t;
    return {b, p, ad.rope_abs ? p : t};
  }
  return {ad.seq[i], ad.pos[i], ad.rope[i]};
}

// Decode: cache row, attended length (causal: position + 1), RoPE row of row r.
__device__ __forceinline__ TokAddr row_addr(const Addressing& ad, int r) {
  if (ad.start_pos) {
    const int b = ad.T == 1 ? r : r / ad.T, t = r - b * ad.T;
    const int p = ad.start_pos[b] + t;
    return {b, p + 1, ad.rope_abs ? p : t};
  }
  return {ad.seq[r], ad.pos[r], ad.rope[r]};
}

__device__ __forceinline__ int row_len(const Addressing& ad, int r) {
  if (ad.start_pos) {
    const int b = r / ad.T;
    return ad.start_pos[b] + (r - b * ad.T) + 1;
  }
  return ad.pos[r];
}

// Attended length of query row r as the decode kernel uses it: clamped to the
// cache, 0 for a row whose cache row is out of range.
// Reads the cache-row and length arrays only (explicit mode) or start_pos.
__device__ __forceinline__ int clamped_row_len(const Addressing& ad, int r, int64_t cache_b, int64_t cache_s) {
  const int b = ad.start_pos ? r / ad.T : ad.seq[r];
  int L = row_len(ad, r);
  if (L > cache_s) L = static_cast<int>(cache_s);
  if (b < 0 || b >= cache_b) L = 0;
  return L;
}

// ---------------------------------------------------------------------------
// Device side of the balanced plan: every wave of a workgroup computes it
// from the rows' lengths (lane l holds rows PER*l .. PER*l + PER - 1), then
// finds the (row, split) of workgroup `bid` in the row-major order of all
// rows' splits.  Cross-lane sums, maxima and the prefix scan use DPP (no LDS
// round trips): this runs ahead of every workgroup's first load.
// ---------------------------------------------------------------------------
struct BalancedSlot {
  int r, split, chunk;
  bool ok;       // false: bid is past the plan's last workgroup
  TokAddr addr;  // row_addr of row r, read with the plan's loads
};

// Inclusive prefix over the 64 lanes with DPP, for sums or maxima of
// non-negative values (0, which lanes shifted in from outside a row read, is
// the identity of both): Hillis-Steele within each 16-lane row (row_shr 1, 2,
// 4, 8), then row 0's last lane into row 1 and row 2's into row 3
// (row_bcast:15), then lane 31 into rows 2 and 3 (row_bcast:31).  Lane 63
// ends with the wave's total.
template <bool MAX>
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  auto op = [](int a, int b) { return MAX ? (a > b ? a : b) : a + b; };
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true));
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true));
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true));
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true));
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));
  return x;
}
__device__ __forceinline__ int wave_total(int x) {
  return __builtin_amdgcn_readlane(wave_inclusive_scan<false>(x), 63);
}
__device__ __forceinline__ int wave_max_nonneg(int x) {
  return __builtin_amdgcn_readlane(wave_inclusive_scan<true>(x), 63);
}

// Branch-free: every lane loads its rows (indices clamped into the batch)
// and masks what lies past n_rows.
template <int PER>
__device__ __forceinline__ BalancedSlot balanced_slot_t(const Addressing& ad, int n_rows, int64_t cache_b,
                                                        int64_t cache_s, int n_splits, int min_chunk, int target,
                                                        int bid) {
  const int lane = threadIdx.x & 63;
  int lt[PER];
  bool valid[PER];
  TokAddr ta[PER];
  int mine_tiles = 0, mx = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int r = PER * lane + j;
    valid[j] = r < n_rows;
    ta[j] = row_addr(ad, valid[j] ? r : n_rows - 1);
    int L = ta[j].pos;  // clamped as clamped_row_len does
    L = L > cache_s ? static_cast<int>(cache_s) : L;
    L = (ta[j].b < 0 || ta[j].b >= cache_b || !valid[j]) ? 0 : L;
    lt[j] = L > 0 ? (L >> 6) + ((L & 63) != 0) : 0;  // < 2^18
    mine_tiles += lt[j];
    mx = lt[j] > mx ? lt[j] : mx;
  }
  const int sum = wave_total(mine_tiles);  // < 2^26
  mx = wave_max_nonneg(mx);
  int cnt[PER];
  // Workgroups of this lane's rows at chunk ct (tiles): an empty row takes one.
  auto lane_blocks = [&](int ct) {
    int n = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int q = ceil_div_small(lt[j], ct);
      cnt[j] = valid[j] ? (q > 1 ? q : 1) : 0;
      n += cnt[j];
    }
    return n;
  };
  int lo, hi;
  balanced_bounds(sum, mx, n_rows, n_splits, min_chunk, target, &lo, &hi);
  while (lo < hi) {  // uniform
    const int mid = lo + (hi - lo) / 2;
    if (wave_total(lane_blocks(mid)) <= target) hi = mid;
    else lo = mid + 1;
  }
  const int ct = lo;
  const int mine = lane_blocks(ct);
  const int incl = wave_inclusive_scan<false>(mine);
  const int excl = incl - mine;
  const bool here = bid >= excl && bid < incl;
  const uint64_t who = __ballot(here);
  BalancedSlot out{0, 0, 64 * ct, who != 0, TokAddr{0, 0, 0}};
  if (!out.ok) return out;
  int rr = 0, sp = 0;
  TokAddr t{0, 0, 0};
  int off = bid - excl;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const bool hit = off >= 0 && off < cnt[j];
    rr = hit ? PER * lane + j : rr;
    sp = hit ? off : sp;
    t.b = hit ? ta[j].b : t.b;  // field by field: a select of the structs goes through memory
    t.pos = hit ? ta[j].pos : t.pos;
    t.rope = hit ? ta[j].rope : t.rope;
    off -= cnt[j];
  }
  const int src = static_cast<int>(__ffsll(static_cast<unsigned long long>(who))) - 1;  // uniform
  out.r = __builtin_amdgcn_readlane(rr, src);
  out.split = __builtin_amdgcn_readlane(sp, src);
  out.addr = TokAddr{__builtin_amdgcn_readlane(t.b, src), __builtin_amdgcn_readlane(t.pos, src),
                     __builtin_amdgcn_readlane(t.rope, src)};
  return out;
}

__device__ __forceinline__ BalancedSlot balanced_slot(const Addressing& ad, int n_rows, int64_t cache_b,
                                                      int64_t cache_s, int n_splits, int min_chunk, int target,
                                                      int bid) {
  if (n_rows <= 64) return balanced_slot_t<1>(ad, n_rows, cache_b, cache_s, n_splits, min_chunk, target, bid);
  return balanced_slot_t<kBalanceMaxRows / 64>(ad, n_rows, cache_b, cache_s, n_splits, min_chunk, target, bid);
}

// Runs f(std::integral_constant<int, NB>) for the instance of a latent row
// of R channels (NB = ceil(R / 64), 1..kMaxNB); -1 when R is out of range.
template <typename F>
int with_nb(int R, F&& f) {
  switch ((R + 63) / 64) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 5: return f(std::integral_constant<int, 5>{});
    case 6: return f(std::integral_constant<int, 6>{});
    case 7: return f(std::integral_constant<int, 7>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default: return -1;
  }
}

// with_nb over NB = 1..kMaxNBWide (ranks up to 1024), for the kernels built
// that wide.
template <typename F>
int with_nb_wide(int R, F&& f) {
  const int nb = (R + 63) / 64;
  if (nb <= kMaxNB) return with_nb(R, f);
  switch (nb) {
    case 9: return f(std::integral_constant<int, 9>{});
    case 10: return f(std::integral_constant<int, 10>{});
    case 11: return f(std::integral_constant<int, 11>{});
    case 12: return f(std::integral_constant<int, 12>{});
    case 13: return f(std::integral_constant<int, 13>{});
    case 14: return f(std::integral_constant<int, 14>{});
    case 15: return f(std::integral_constant<int, 15>{});
    case 16: return f(std::integral_constant<int, 16>{});
    default: return -1;
  }
}

}  // namespace swamla
