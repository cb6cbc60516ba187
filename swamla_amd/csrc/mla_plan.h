// mla_plan.h — split plan and token / row addressing shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
    const int b = r / ad.T, t = r - b * ad.T;
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

}  // namespace swamla
