// mla_abi.cpp — the extern "C" boundary: argument validation, error
// reporting and dispatch to the gfx950 launchers.  Validation never touches
// the GPU, so every error path is testable on a machine without one.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/swamla_mi355x.h"
#include "../../include/swamla_mi355x_testing.h"
#include "mla_args.h"
#include "mla_plan.h"
#include "mla_scratch.h"
#include "numerics.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return SWAMLA_OK;
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

// allow32: the entry point also runs 32 heads in one launch.  Ranks above
// 64 kMaxNB are built for the append, the merge and the decode attention
// (VALU kernel); the other entry points return UNSUPPORTED for them.
int check_geometry(int32_t H, int32_t R, int32_t P, bool allow32 = false) {
  if ((H != 16 && !(allow32 && H == 32)) || P != 64 || R < 1 || R > 64 * swamla::kMaxNBWide)
    return fail(SWAMLA_ERR_UNSUPPORTED,
                "unsupported geometry H=%d R=%d P=%d (this build: H=16%s, P=64, 1 <= R <= %d)", H, R, P,
                allow32 ? " or 32" : "", 64 * swamla::kMaxNBWide);
  return SWAMLA_OK;
}

// Bytes a lane of the append arithmetic moves at once: its R_pad / 64 bf16
// channels, as the widest power of two dividing them (at least 4: the k_pe
// pair is one 4-byte word), at most 16.
uintptr_t lane_align(int32_t R) {
  const int b = 2 * (swamla::padded_rank(R) / 64);
  uintptr_t a = 16;
  while (a > 4 && b % a != 0) a >>= 1;
  return a;
}

// Element size of the model (query/output/k_pe) dtype; 0 if not a model dtype.
int model_elem(int32_t dt) { return dt == SWAMLA_DTYPE_F32 ? 4 : (dt == SWAMLA_DTYPE_BF16 ? 2 : 0); }

int check_pair(int32_t dt, int32_t cdt) {
  const bool okp = (dt == SWAMLA_DTYPE_BF16 && (cdt == SWAMLA_DTYPE_BF16 || cdt == SWAMLA_DTYPE_FP8)) ||
                   (dt == SWAMLA_DTYPE_F32 && cdt == SWAMLA_DTYPE_F32);
  if (!okp)
    return fail(SWAMLA_ERR_UNSUPPORTED,
                "unsupported dtype pair model=%d cache=%d (built: bf16/bf16, bf16/fp8, f32/f32)", dt,
                cdt);
  return SWAMLA_OK;
}

int hip_fail(const char* what) {
  const hipError_t e = hipGetLastError();
  return fail(SWAMLA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
}


int mla_abi_version_impl() { return SWAMLA_ABI_VERSION; }

const char* last_error_impl() { return g_err; }

// The kernels' own plan (mla_plan.h), one definition for host and device.
int32_t split_count_impl(int32_t L, int32_t n_splits, int32_t min_chunk) {
  if (n_splits < 1 || min_chunk < 1) return 0;
  return swamla::split_count(L, n_splits, min_chunk);
}

// Addressing: explicit per-entry arrays, or dense (start_pos[n / T]).
int check_addressing(const char* fn, int32_t n, const int32_t* a0, const int32_t* a1, const int32_t* a2,
                     const int32_t* start_pos, int32_t T, bool need_a0, bool need_a2,
                     swamla::Addressing* ad, int32_t rope_abs) {
  if (start_pos) {
    if (a0 || a1 || a2)
      return fail(SWAMLA_ERR_INVALID_ARG, "%s: pass either start_pos or the per-entry arrays, not both", fn);
    if (T < 1) return fail(SWAMLA_ERR_INVALID_ARG, "%s: entries per sequence %d < 1", fn, T);
    if (n % T != 0) return fail(SWAMLA_ERR_INVALID_ARG, "%s: %d entries is not a multiple of %d", fn, n, T);
    if (rope_abs != 0 && rope_abs != 1) return fail(SWAMLA_ERR_INVALID_ARG, "%s: rope_abs must be 0 or 1", fn);
  } else if (n > 0 && ((need_a0 && !a0) || !a1 || (need_a2 && !a2))) {
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: null per-entry index array", fn);
  }
  *ad = swamla::Addressing{a0, a1, a2, start_pos, start_pos ? T : 1, rope_abs};
  return SWAMLA_OK;
}

}  // namespace

extern "C" {

int mla_abi_version(void) { return mla_abi_version_impl(); }

const char* mla_last_error(void) { return last_error_impl(); }

int32_t mla_split_count(int32_t L, int32_t n_splits, int32_t min_chunk) {
  return split_count_impl(L, n_splits, min_chunk);
}

int32_t mla_decode_blocks_per_cu(int32_t dtype, int32_t cache_dtype, int32_t R, int32_t fused) {
  if (int e = check_geometry(16, R, 64)) return e;
  if (int e = check_pair(dtype, cache_dtype)) return e;
  if (fused != 0 && fused != 1) return fail(SWAMLA_ERR_INVALID_ARG, "mla_decode_blocks_per_cu: fused must be 0 or 1");
  int n = 0;
  const int rc = swamla::decode_blocks_per_cu(dtype, cache_dtype, R, fused != 0, &n);
  if (rc == -1)
    return fail(SWAMLA_ERR_UNSUPPORTED, "mla_decode_blocks_per_cu: no decode kernel for model=%d cache=%d fused=%d",
                dtype, cache_dtype, fused);
  if (rc != 0) {
    const hipError_t e = hipGetLastError();
    return fail(SWAMLA_ERR_HIP, "mla_decode_blocks_per_cu: occupancy query failed: %s", hipGetErrorString(e));
  }
  return n;
}

int32_t mla_balanced_chunk(const int32_t* lens, int32_t n_rows, int32_t n_splits, int32_t min_chunk,
                           int32_t balance_blocks) {
  if (n_rows < 0 || n_rows > swamla::kBalanceMaxRows || (n_rows > 0 && !lens) || n_splits < 1 ||
      n_splits > 1024 || min_chunk < 1 || balance_blocks < 1 || balance_blocks > 65535 || n_rows > balance_blocks)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_balanced_chunk: bad arguments (n_rows=%d, n_splits=%d, "
                "min_chunk=%d, balance_blocks=%d)", n_rows, n_splits, min_chunk, balance_blocks);
  for (int r = 0; r < n_rows; ++r)
    if (lens[r] > swamla::kBalanceMaxSeq)
      return fail(SWAMLA_ERR_INVALID_ARG, "mla_balanced_chunk: length %d above %lld", lens[r],
                  (long long)swamla::kBalanceMaxSeq);
  return swamla::balanced_chunk_host(lens, n_rows, n_splits, min_chunk, balance_blocks);
}

int mla_append(const void* kv_in, int64_t in_row_stride, int32_t n_tok, const int32_t* seq_idx,
               const int32_t* dst_pos, const int32_t* rope_pos, const int32_t* start_pos,
               int32_t tokens_per_seq, int32_t rope_abs, const void* ln_w, const void* ln_b, float eps,
               const void* cos_tab, const void* sin_tab, int64_t rope_len, void* ckv_cache,
               void* kpe_cache, float* ckv_scale, int64_t cache_batch, int64_t cache_seq,
               int32_t* err_flag, int32_t in_dtype, int32_t cache_dtype, int32_t R, int32_t P,
               void* stream) {
  if (int e = check_geometry(16, R, P)) return e;
  if (int e = check_pair(in_dtype, cache_dtype)) return e;
  if (n_tok < 0) return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: n_tok=%d < 0", n_tok);
  if (n_tok > (1 << 30)) return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: n_tok=%d too large", n_tok);
  if (!ckv_cache || !kpe_cache || !ln_w || !ln_b || !cos_tab || !sin_tab)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: null cache / LayerNorm / RoPE pointer");
  if (n_tok > 0 && !kv_in) return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: null input rows");
  swamla::Addressing ad;
  if (int e = check_addressing("mla_append", n_tok, seq_idx, dst_pos, rope_pos, start_pos, tokens_per_seq,
                               true, true, &ad, rope_abs))
    return e;
  if (cache_dtype == SWAMLA_DTYPE_FP8 && !ckv_scale)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: fp8 cache needs ckv_scale");
  const int RP = swamla::padded_rank(R);
  if (in_row_stride < RP + P)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: in_row_stride=%lld < R_pad+P=%d",
                (long long)in_row_stride, RP + P);
  if (cache_batch < 1 || cache_seq < 1 || cache_seq > (int64_t(1) << 31) - 1)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: bad cache shape [%lld, %lld]",
                (long long)cache_batch, (long long)cache_seq);
  if (rope_len < 1) return fail(SWAMLA_ERR_INVALID_ARG, "mla_append: rope_len=%lld < 1", (long long)rope_len);
  const int es = model_elem(in_dtype);
  if (!aligned(ckv_cache, 16) || !aligned(kpe_cache, es) || (kv_in && !aligned(kv_in, es)) ||
      !aligned(ln_w, es) || !aligned(ln_b, es) || !aligned(cos_tab, es) || !aligned(sin_tab, es) ||
      (ckv_scale && !aligned(ckv_scale, 4)))
    return fail(SWAMLA_ERR_MISALIGNED, "mla_append: ckv_cache must be 16-byte aligned, others element-aligned");
  swamla::AppendArgs a{kv_in,    in_row_stride, n_tok,     R,           ad,        ln_w,    ln_b,    eps,
                       cos_tab,  sin_tab,       rope_len,  ckv_cache,   kpe_cache, ckv_scale,
                       cache_batch, cache_seq,  err_flag};
  const int rc = swamla::launch_append(a, in_dtype, cache_dtype, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_append: no kernel for this dtype pair and rank");
  if (rc != 0) return hip_fail("mla_append");
  return ok();
}

}  // extern "C"

namespace {

// Validation shared by mla_decode_attn and mla_decode_attn_append; fills *a.
int check_decode(const char* fn, const void* q_abs, int64_t q_abs_rs, int64_t q_abs_hs, const void* q_pe,
                 int64_t q_pe_rs, int64_t q_pe_hs, const void* cos_tab, const void* sin_tab, int64_t rope_len,
                 const void* ckv_cache, const void* kpe_cache, const float* ckv_scale, int64_t cache_batch,
                 int64_t cache_seq, const int32_t* row_seq, const int32_t* kv_len, const int32_t* q_rope_pos,
                 const int32_t* start_pos, int32_t rows_per_seq, int32_t rope_abs, int32_t n_rows, int32_t H,
                 int32_t R, int32_t P, float sm_scale, int32_t n_splits, int32_t min_chunk, int32_t balance,
                 int32_t* plan, float* o_part, float* lse_part, void* o_lat, int64_t o_rs, int64_t o_hs,
                 float* lse_out, int32_t dtype, int32_t cache_dtype, swamla::DecodeArgs* a,
                 int32_t max_rows = 65535, bool allow32 = false) {
  if (int e = check_geometry(H, R, P, allow32)) return e;
  if (H == 32 && (dtype != SWAMLA_DTYPE_BF16 || swamla::padded_rank(R) > 256))
    return fail(SWAMLA_ERR_UNSUPPORTED,
                "%s: 32 heads in one launch are built for a bf16 model with kv_lora_rank <= 256", fn);
  if (int e = check_pair(dtype, cache_dtype)) return e;
  if (n_rows < 0 || n_rows > max_rows)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: n_rows=%d outside [0, %d]", fn, n_rows, max_rows);
  if (n_splits < 1 || n_splits > 1024)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: n_splits=%d outside [1, 1024]", fn, n_splits);
  if (min_chunk < 1) return fail(SWAMLA_ERR_INVALID_ARG, "%s: min_chunk=%d < 1", fn, min_chunk);
  if (balance < 0 || balance > 65535)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: balance_blocks=%d outside [0, 65535]", fn, balance);
  if (balance > 0 && (n_rows > balance || n_rows > swamla::kBalanceMaxRows))
    return fail(SWAMLA_ERR_INVALID_ARG,
                "%s: a balanced plan needs n_rows <= balance_blocks and n_rows <= %d (n_rows=%d, "
                "balance_blocks=%d)", fn, swamla::kBalanceMaxRows, n_rows, balance);
  if (balance > 0 && cache_seq > swamla::kBalanceMaxSeq)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: a balanced plan covers caches of at most %lld positions", fn,
                (long long)swamla::kBalanceMaxSeq);
  if (plan && !aligned(plan, 4)) return fail(SWAMLA_ERR_MISALIGNED, "%s: plan must be 4-byte aligned", fn);
  if (!(sm_scale > 0.f)) return fail(SWAMLA_ERR_INVALID_ARG, "%s: sm_scale must be > 0", fn);
  if (!ckv_cache || !kpe_cache || !cos_tab || !sin_tab || !o_lat)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: null cache / RoPE / output pointer", fn);
  if (n_rows > 0 && (!q_abs || !q_pe)) return fail(SWAMLA_ERR_INVALID_ARG, "%s: null query pointer", fn);
  swamla::Addressing ad;
  if (int e = check_addressing(fn, n_rows, row_seq, kv_len, q_rope_pos, start_pos, rows_per_seq, true, true,
                               &ad, rope_abs))
    return e;
  if (n_splits > 1 && (!o_part || !lse_part))
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: n_splits > 1 needs o_part and lse_part", fn);
  if (cache_dtype == SWAMLA_DTYPE_FP8 && !ckv_scale)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: fp8 cache needs ckv_scale", fn);
  if (cache_batch < 1 || cache_seq < 1 || cache_seq > (int64_t(1) << 31) - 1 || rope_len < 1)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: bad cache / rope table shape", fn);
  const int RP = swamla::padded_rank(R);
  if (q_abs_hs < RP || q_pe_hs < P || o_hs < RP || q_abs_rs < 0 || q_pe_rs < 0 || o_rs < 0)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: head strides must cover R_pad / P values", fn);
  if (dtype == SWAMLA_DTYPE_BF16) {
    // 16-byte vector loads / stores of 8 bf16.
    if (!aligned(q_abs, 16) || !aligned(q_pe, 16) || !aligned(o_lat, 16) || !aligned(ckv_cache, 16) ||
        !aligned(kpe_cache, 16) || !aligned(cos_tab, 8) || !aligned(sin_tab, 8) ||
        (q_abs_rs | q_abs_hs | q_pe_rs | q_pe_hs | o_rs | o_hs) % 8 != 0)
      return fail(SWAMLA_ERR_MISALIGNED,
                  "%s: bf16 operands need 16-byte aligned bases (RoPE tables: 8-byte) and strides "
                  "that are multiples of 8 elements", fn);
  } else {
    if (!aligned(q_abs, 4) || !aligned(q_pe, 4) || !aligned(o_lat, 16) || !aligned(ckv_cache, 4) ||
        !aligned(kpe_cache, 4) || !aligned(cos_tab, 4) || !aligned(sin_tab, 4) || (o_rs | o_hs) % 4 != 0)
      return fail(SWAMLA_ERR_MISALIGNED,
                  "%s: fp32 output needs a 16-byte aligned base and strides that are "
                  "multiples of 4", fn);
  }
  if ((o_part && !aligned(o_part, 16)) || (lse_part && !aligned(lse_part, 4)) ||
      (ckv_scale && !aligned(ckv_scale, 4)) || (lse_out && !aligned(lse_out, 4)))
    return fail(SWAMLA_ERR_MISALIGNED, "%s: o_part must be 16-byte aligned, lse / scale arrays 4-byte", fn);
  const float log2e = 1.4426950408889634f;
  *a = swamla::DecodeArgs{R,         q_abs,     q_abs_rs,  q_abs_hs,  q_pe,      q_pe_rs,     q_pe_hs,
                          cos_tab,   sin_tab,   rope_len,  ckv_cache, kpe_cache,   ckv_scale,
                          cache_batch, cache_seq, ad,      n_rows,    sm_scale * log2e, n_splits,
                          min_chunk, balance,   plan,      o_part,    lse_part,  o_lat,
                          o_rs,      o_hs,      lse_out,   swamla::AppendArgs{}};
  a->H = H;
  return SWAMLA_OK;
}

}  // namespace

extern "C" {

int mla_decode_attn(const void* q_abs, int64_t q_abs_rs, int64_t q_abs_hs, const void* q_pe,
                    int64_t q_pe_rs, int64_t q_pe_hs, const void* cos_tab, const void* sin_tab,
                    int64_t rope_len, const void* ckv_cache, const void* kpe_cache,
                    const float* ckv_scale, int64_t cache_batch, int64_t cache_seq,
                    const int32_t* row_seq, const int32_t* kv_len, const int32_t* q_rope_pos,
                    const int32_t* start_pos, int32_t rows_per_seq, int32_t rope_abs, int32_t n_rows,
                    int32_t H, int32_t R, int32_t P, float sm_scale, int32_t n_splits,
                    int32_t min_chunk, int32_t balance_blocks, int32_t* plan, float* o_part,
                    float* lse_part, void* o_lat, int64_t o_rs, int64_t o_hs, float* lse_out,
                    int32_t dtype, int32_t cache_dtype, void* stream) {
  swamla::DecodeArgs a;
  if (int e = check_decode("mla_decode_attn", q_abs, q_abs_rs, q_abs_hs, q_pe, q_pe_rs, q_pe_hs, cos_tab,
                           sin_tab, rope_len, ckv_cache, kpe_cache, ckv_scale, cache_batch, cache_seq, row_seq,
                           kv_len, q_rope_pos, start_pos, rows_per_seq, rope_abs, n_rows, H, R, P, sm_scale,
                           n_splits, min_chunk, balance_blocks, plan, o_part, lse_part, o_lat, o_rs, o_hs, lse_out,
                           dtype, cache_dtype, &a, 65535, true))
    return e;
  const int rc = swamla::launch_decode(a, dtype, cache_dtype, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_decode_attn: no kernel for this dtype pair, head count and rank");
  if (rc != 0) return hip_fail("mla_decode_attn");
  return ok();
}

int mla_decode_attn_append(const void* kv_in, int64_t in_row_stride, const void* ln_w, const void* ln_b,
                           float eps, int32_t* err_flag, const void* q_abs, int64_t q_abs_rs,
                           int64_t q_abs_hs, const void* q_pe, int64_t q_pe_rs, int64_t q_pe_hs,
                           const void* cos_tab, const void* sin_tab, int64_t rope_len, void* ckv_cache,
                           void* kpe_cache, float* ckv_scale, int64_t cache_batch, int64_t cache_seq,
                           const int32_t* start_pos, int32_t rope_abs, int32_t n_rows, int32_t H, int32_t R,
                           int32_t P, float sm_scale, int32_t n_splits, int32_t min_chunk,
                           int32_t balance_blocks, int32_t* plan, float* o_part, float* lse_part, void* o_lat,
                           int64_t o_rs, int64_t o_hs, float* lse_out, int32_t dtype, int32_t cache_dtype,
                           void* stream) {
  const char* fn = "mla_decode_attn_append";
  if (dtype != SWAMLA_DTYPE_BF16)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: model dtype %d not built (bf16 only)", fn, dtype);
  if (!start_pos) return fail(SWAMLA_ERR_INVALID_ARG, "%s: needs dense addressing (start_pos)", fn);
  swamla::DecodeArgs a;
  if (int e = check_decode(fn, q_abs, q_abs_rs, q_abs_hs, q_pe, q_pe_rs, q_pe_hs, cos_tab, sin_tab, rope_len,
                           ckv_cache, kpe_cache, ckv_scale, cache_batch, cache_seq, nullptr, nullptr, nullptr,
                           start_pos, 1, rope_abs, n_rows, H, R, P, sm_scale, n_splits, min_chunk,
                           balance_blocks, plan, o_part, lse_part, o_lat, o_rs, o_hs, lse_out, dtype, cache_dtype,
                           &a, 65535, true))
    return e;
  if (n_rows > 0 && !kv_in) return fail(SWAMLA_ERR_INVALID_ARG, "%s: null input rows", fn);
  if (!ln_w || !ln_b) return fail(SWAMLA_ERR_INVALID_ARG, "%s: null LayerNorm pointer", fn);
  const int RP = swamla::padded_rank(R);
  if (in_row_stride < RP + P)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: in_row_stride=%lld < R_pad+P=%d", fn, (long long)in_row_stride,
                RP + P);
  // a lane reads its R_pad / 64 channels of the row and of the LayerNorm
  // parameters at once
  const uintptr_t la = lane_align(R);
  if ((kv_in && !aligned(kv_in, la)) || in_row_stride % (la / 2) != 0 || !aligned(ln_w, la) || !aligned(ln_b, la) ||
      !aligned(cos_tab, 2) || !aligned(sin_tab, 2))
    return fail(SWAMLA_ERR_MISALIGNED,
                "%s: input rows and LayerNorm parameters need %d-byte aligned bases and a row stride that is a "
                "multiple of %d elements", fn, static_cast<int>(la), static_cast<int>(la / 2));
  if (n_rows == 0) return ok();
  a.fa = swamla::AppendArgs{kv_in,   in_row_stride, n_rows,      R,         a.ad,      ln_w,      ln_b,   eps,
                            cos_tab, sin_tab,       rope_len,    ckv_cache, kpe_cache, ckv_scale,
                            cache_batch, cache_seq, err_flag};
  const int rc = swamla::launch_decode(a, dtype, cache_dtype, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: no kernel for this dtype pair, head count and rank", fn);
  if (rc != 0) return hip_fail(fn);
  return ok();
}

int mla_decode_attn_noalloc(const void* q_abs, int64_t q_abs_rs, int64_t q_abs_hs, const void* q_pe,
                            int64_t q_pe_rs, int64_t q_pe_hs, const void* cos_tab, const void* sin_tab,
                            int64_t rope_len, const void* ckv_cache, const void* kpe_cache,
                            const float* ckv_scale, int64_t cache_batch, int64_t cache_seq,
                            const int32_t* row_seq, const int32_t* kv_len, const int32_t* q_rope_pos,
                            const int32_t* start_pos, int32_t rows_per_seq, int32_t rope_abs, int32_t n_rows,
                            int32_t H, int32_t R, int32_t P, float sm_scale, int32_t n_splits,
                            int32_t min_chunk, int32_t balance_blocks, void* o_lat, int64_t o_rs, int64_t o_hs,
                            float* lse_out, int32_t dtype, int32_t cache_dtype, void* stream) {
  const char* fn = "mla_decode_attn_noalloc";
  if (int e = check_geometry(H, R, P)) return e;
  if (n_rows < 0 || n_rows > 65535 || n_splits < 1 || n_splits > 1024)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: n_rows=%d / n_splits=%d outside [0, 65535] / [1, 1024]", fn, n_rows,
                n_splits);
  // partials of every (row, split, head): R_pad fp32 values and one log-sum-exp
  const int64_t part = n_splits > 1 ? int64_t(n_rows) * n_splits * H * swamla::padded_rank(R) * 4 : 0;
  if (part > static_cast<int64_t>(swamla::kScratchPartBytes))
    return fail(SWAMLA_ERR_UNSUPPORTED,
                "%s: %d rows x %d splits need %lld bytes of split partials, above this entry point's fixed "
                "scratch of %lld bytes (use fewer splits or rows per call, or mla_decode_attn with a workspace)",
                fn, n_rows, n_splits, (long long)part, (long long)swamla::kScratchPartBytes);
  // Validate everything first (no GPU call), with stand-ins for the
  // scratch pointers: 256-aligned, as the real area is.
  float* const stand_in = reinterpret_cast<float*>(uintptr_t(256));
  swamla::DecodeArgs a;
  if (int e = check_decode(fn, q_abs, q_abs_rs, q_abs_hs, q_pe, q_pe_rs, q_pe_hs, cos_tab, sin_tab, rope_len,
                           ckv_cache, kpe_cache, ckv_scale, cache_batch, cache_seq, row_seq, kv_len, q_rope_pos,
                           start_pos, rows_per_seq, rope_abs, n_rows, H, R, P, sm_scale, n_splits, min_chunk,
                           balance_blocks, nullptr, stand_in, stand_in, o_lat, o_rs, o_hs, lse_out, dtype,
                           cache_dtype, &a))
    return e;
  swamla::ScratchUse use(stream);
  if (use.status == -2) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: device ordinal beyond the scratch table", fn);
  if (use.status != 0)
    return fail(SWAMLA_ERR_HIP, "%s: scratch set-up failed: %s", fn, hipGetErrorString(hipGetLastError()));
  uint8_t* const base = static_cast<uint8_t*>(use.area);
  float* const o_part = reinterpret_cast<float*>(base);
  float* const lse_part = reinterpret_cast<float*>(base + swamla::kScratchPartBytes);
  int32_t* const plan = balance_blocks > 0 ? reinterpret_cast<int32_t*>(base + swamla::kScratchPlanOffset) : nullptr;
  a.o_part = o_part;
  a.lse_part = lse_part;
  a.plan = plan;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = swamla::launch_decode(a, dtype, cache_dtype, st);
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: no kernel for this dtype pair, head count and rank", fn);
  if (rc != 0) return hip_fail(fn);
  if (n_splits == 1 || n_rows == 0) {
    use.launched();
    return ok();
  }
  // every partial the merge reads was written by the launch above
  swamla::MergeArgs m{o_part, lse_part, a.ad, cache_batch, cache_seq, n_rows, n_splits,
                      min_chunk, plan, R, o_lat, o_rs, o_hs, lse_out};
  rc = swamla::launch_merge(m, dtype, st);
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: no merge kernel for dtype %d", fn, dtype);
  if (rc != 0) return hip_fail(fn);
  use.launched();
  return ok();
}

int mla_prefill_attn(const void* q_abs, int64_t q_abs_rs, int64_t q_abs_hs, const void* q_pe, int64_t q_pe_rs,
                     int64_t q_pe_hs, const void* cos_tab, const void* sin_tab, int64_t rope_len,
                     const void* ckv_cache, const void* kpe_cache, const float* ckv_scale, int64_t cache_batch,
                     int64_t cache_seq, const int32_t* start_pos, int32_t tokens_per_seq, int32_t rope_abs,
                     int32_t n_rows, int32_t H, int32_t R, int32_t P, float sm_scale, void* o_lat, int64_t o_rs,
                     int64_t o_hs, int32_t dtype, int32_t cache_dtype, void* stream) {
  const char* fn = "mla_prefill_attn";
  if (dtype != SWAMLA_DTYPE_BF16)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: model dtype %d not built (bf16 only)", fn, dtype);
  if (!start_pos) return fail(SWAMLA_ERR_INVALID_ARG, "%s: needs dense addressing (start_pos)", fn);
  if (swamla::padded_rank(R) > 256)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: kv_lora_rank %d above 256 (the per-row mla_decode_attn path serves it)",
                fn, R);
  swamla::DecodeArgs a;
  if (int e = check_decode(fn, q_abs, q_abs_rs, q_abs_hs, q_pe, q_pe_rs, q_pe_hs, cos_tab, sin_tab, rope_len,
                           ckv_cache, kpe_cache, ckv_scale, cache_batch, cache_seq, nullptr, nullptr, nullptr,
                           start_pos, tokens_per_seq, rope_abs, n_rows, H, R, P, sm_scale, 1, 1, 0, nullptr,
                           nullptr, nullptr, o_lat, o_rs, o_hs, nullptr, dtype, cache_dtype, &a, 1 << 30))
    return e;
  // grid: (ceil(T / 4), sequences)
  if (n_rows / tokens_per_seq > 65535)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: %d sequences exceed 65535", fn, n_rows / tokens_per_seq);
  const int rc = swamla::launch_prefill(a, dtype, cache_dtype, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: no kernel for this dtype pair, head count and rank", fn);
  if (rc != 0) return hip_fail(fn);
  return ok();
}

int mla_merge(const float* o_part, const float* lse_part, const int32_t* row_seq, const int32_t* kv_len,
              const int32_t* start_pos, int32_t rows_per_seq, int64_t cache_batch, int64_t cache_seq,
              int32_t n_rows, int32_t H, int32_t R, int32_t n_splits, int32_t min_chunk, const int32_t* plan,
              void* o_lat, int64_t o_rs, int64_t o_hs, float* lse_out, int32_t dtype, void* stream) {
  if (int e = check_geometry(H, R, 64, true)) return e;
  if (!model_elem(dtype)) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_merge: dtype %d not built", dtype);
  if (n_rows < 0 || n_rows > 65535)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge: n_rows=%d outside [0, 65535]", n_rows);
  if (n_splits < 1 || n_splits > 1024)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge: n_splits=%d outside [1, 1024]", n_splits);
  if (min_chunk < 1) return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge: min_chunk=%d < 1", min_chunk);
  if (n_splits == 1 || n_rows == 0) return ok();  // nothing to merge
  swamla::Addressing ad;
  if (int e = check_addressing("mla_merge", n_rows, row_seq, kv_len, nullptr, start_pos, rows_per_seq, true,
                               false, &ad, 0))
    return e;
  if (cache_batch < 1 || cache_seq < 1 || cache_seq > (int64_t(1) << 31) - 1)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge: bad cache shape");
  if (!o_part || !lse_part || !o_lat) return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge: null pointer");
  if (o_hs < swamla::padded_rank(R) || o_rs < 0) return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge: bad output strides");
  // a lane writes 4 channels: 16 B (fp32) or 8 B (bf16)
  if (!aligned(o_part, 16) || !aligned(o_lat, dtype == SWAMLA_DTYPE_F32 ? 16 : 8) || (o_rs | o_hs) % 4 != 0 ||
      (plan && !aligned(plan, 4)))
    return fail(SWAMLA_ERR_MISALIGNED, "mla_merge: misaligned partials, plan or output");
  swamla::MergeArgs a{o_part, lse_part, ad,   cache_batch, cache_seq, n_rows, n_splits,
                      min_chunk, plan, R, o_lat, o_rs, o_hs, lse_out};
  a.H = H;
  const int rc = swamla::launch_merge(a, dtype, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_merge: no kernel for dtype %d", dtype);
  if (rc != 0) return hip_fail("mla_merge");
  return ok();
}

int mla_linear(const void* x, int64_t x_rs, int64_t x_bs, const void* w, int64_t w_rs, int64_t w_bs,
               const void* bias, int64_t bias_bs, void* y, int64_t y_rs, int64_t y_bs, int32_t M,
               int32_t N, int32_t K, int32_t batch, int32_t dtype, void* stream) {
  if (dtype != SWAMLA_DTYPE_BF16) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_linear: dtype %d not built (bf16 only)", dtype);
  if (M < 0 || M > 128) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_linear: M=%d outside [0, 128]", M);
  if (N < 0 || N % 16 != 0) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_linear: N=%d is not a multiple of 16", N);
  if (K < 128 || K % 128 != 0) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_linear: K=%d is not a positive multiple of 128", K);
  if (batch < 0 || batch > 65535) return fail(SWAMLA_ERR_INVALID_ARG, "mla_linear: batch=%d outside [0, 65535]", batch);
  if (N / 16 > 65535) return fail(SWAMLA_ERR_INVALID_ARG, "mla_linear: N=%d too large", N);
  if (M == 0 || N == 0 || batch == 0) return ok();
  if (!x || !w || !y) return fail(SWAMLA_ERR_INVALID_ARG, "mla_linear: null x / w / y");
  if (x_rs < K || w_rs < K || y_rs < N || x_rs < 0 || x_bs < 0 || w_bs < 0 || y_bs < 0 || bias_bs < 0)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_linear: row strides must cover K (x, w) and N (y)");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 2) || (bias && !aligned(bias, 2)) ||
      (x_rs | x_bs | w_rs | w_bs) % 8 != 0)
    return fail(SWAMLA_ERR_MISALIGNED,
                "mla_linear: x and w need 16-byte aligned bases and strides that are multiples of 8");
  swamla::LinearArgs a{x, x_rs, x_bs, w, w_rs, w_bs, bias, bias_bs, y, y_rs, y_bs, M, N, K};
  const int rc = swamla::launch_linear(a, batch, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_linear: no kernel for M=%d", M);
  if (rc != 0) return hip_fail("mla_linear");
  return ok();
}

int mla_pack_weight(const void* w, int64_t w_rs, int32_t N, int32_t K, void* w_packed, int32_t dtype,
                    void* stream) {
  if (dtype != SWAMLA_DTYPE_BF16)
    return fail(SWAMLA_ERR_UNSUPPORTED, "mla_pack_weight: dtype %d not built (bf16 only)", dtype);
  if (N < 0 || N % 8 != 0) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_pack_weight: N=%d is not a multiple of 8", N);
  if (K < 0 || K % 64 != 0) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_pack_weight: K=%d is not a multiple of 64", K);
  if (N == 0 || K == 0) return ok();
  if (!w || !w_packed) return fail(SWAMLA_ERR_INVALID_ARG, "mla_pack_weight: null pointer");
  if (w_rs < K) return fail(SWAMLA_ERR_INVALID_ARG, "mla_pack_weight: row stride %lld < K=%d", (long long)w_rs, K);
  if (!aligned(w, 16) || !aligned(w_packed, 16) || w_rs % 8 != 0)
    return fail(SWAMLA_ERR_MISALIGNED, "mla_pack_weight: 16-byte aligned bases and a row stride that is a "
                "multiple of 8 are required");
  swamla::PackWeightArgs a{w, w_rs, w_packed, N, K};
  if (swamla::launch_pack_weight(a, static_cast<hipStream_t>(stream)) != 0) return hip_fail("mla_pack_weight");
  return ok();
}

int mla_linear_packed(const void* x, int64_t x_rs, const void* w_packed, const void* bias, void* y, int64_t y_rs,
                      int32_t M, int32_t N, int32_t K, int32_t* advance, int32_t n_advance, int32_t dtype,
                      void* stream) {
  const char* fn = "mla_linear_packed";
  if (dtype != SWAMLA_DTYPE_BF16) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: dtype %d not built (bf16 only)", fn, dtype);
  if (M < 0 || M > 128) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: M=%d outside [0, 128]", fn, M);
  if (N < 0 || N % 8 != 0) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: N=%d is not a multiple of 8", fn, N);
  if (K != 512 && K != 1024 && K != 1536 && K != 2048)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: K=%d (built: 512, 1024, 1536, 2048)", fn, K);
  if (advance && (n_advance < 1 || n_advance > 512 || M == 0 || N == 0))
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: advance needs 1 <= n_advance <= 512 (got %d) and a non-empty product "
                "(M=%d, N=%d)", fn, n_advance, M, N);
  if (M == 0 || N == 0) return ok();
  if (!x || !w_packed || !y) return fail(SWAMLA_ERR_INVALID_ARG, "%s: null x / w_packed / y", fn);
  if (x_rs < K || y_rs < N) return fail(SWAMLA_ERR_INVALID_ARG, "%s: row strides must cover K (x) and N (y)", fn);
  if (advance && !aligned(advance, 4)) return fail(SWAMLA_ERR_MISALIGNED, "%s: advance must be 4-byte aligned", fn);
  if (!aligned(x, 16) || !aligned(w_packed, 16) || x_rs % 8 != 0 || !aligned(y, 2) || (bias && !aligned(bias, 2)))
    return fail(SWAMLA_ERR_MISALIGNED, "%s: x and w_packed need 16-byte aligned bases and x a row stride that is "
                "a multiple of 8", fn);
  swamla::PackedLinearArgs a{x, x_rs, w_packed, bias, y, y_rs, M, N, K, advance, advance ? n_advance : 0};
  const int rc = swamla::launch_linear_packed(a, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: no kernel for M=%d K=%d", fn, M, K);
  if (rc != 0) return hip_fail(fn);
  return ok();
}

int mla_merge_project(const float* o_part, const float* lse_part, const void* o_lat, int64_t o_rs,
                      int64_t o_hs, const int32_t* kv_len, const int32_t* row_seq,
                      const int32_t* start_pos, int32_t rows_per_seq, int64_t cache_batch,
                      int64_t cache_seq, int32_t n_rows, int32_t H, int32_t R, int32_t n_splits,
                      int32_t min_chunk, const int32_t* plan, const void* w, int64_t w_rs, int64_t w_hs,
                      int32_t Dv,
                      void* y, int64_t y_rs, int64_t y_hs, int32_t dtype, void* stream) {
  if (int e = check_geometry(H, R, 64, true)) return e;
  if (swamla::padded_rank(R) > 64 * swamla::kMaxNB)
    return fail(SWAMLA_ERR_UNSUPPORTED, "mla_merge_project: kv_lora_rank %d (built up to %d)", R, 64 * swamla::kMaxNB);
  if (dtype != SWAMLA_DTYPE_BF16)
    return fail(SWAMLA_ERR_UNSUPPORTED, "mla_merge_project: dtype %d not built (bf16 only)", dtype);
  if (Dv != 128) return fail(SWAMLA_ERR_UNSUPPORTED, "mla_merge_project: Dv=%d (this build: 128)", Dv);
  if (n_rows < 0 || n_rows > 65535 * 8)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge_project: n_rows=%d out of range", n_rows);
  if (n_splits < 1 || n_splits > 1024)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge_project: n_splits=%d outside [1, 1024]", n_splits);
  if (min_chunk < 1) return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge_project: min_chunk=%d < 1", min_chunk);
  if (n_rows == 0) return ok();
  swamla::Addressing ad;
  if (int e = check_addressing("mla_merge_project", n_rows, row_seq, kv_len, nullptr, start_pos, rows_per_seq,
                               true, false, &ad, 0))
    return e;
  if (!o_lat || !w || !y) return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge_project: null o_lat / w / y");
  if (n_splits > 1 && (!o_part || !lse_part))
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge_project: n_splits > 1 needs o_part and lse_part");
  if (cache_batch < 1 || cache_seq < 1 || cache_seq > (int64_t(1) << 31) - 1)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge_project: bad cache shape");
  if (o_hs < swamla::padded_rank(R) || w_rs < swamla::padded_rank(R) || y_hs < Dv || o_rs < 0 || w_hs < 0 ||
      y_rs < 0)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_merge_project: strides must cover R_pad / Dv values");
  if (!aligned(o_lat, 16) || !aligned(w, 16) || !aligned(y, 2) || (o_part && !aligned(o_part, 16)) ||
      (lse_part && !aligned(lse_part, 4)) || (plan && !aligned(plan, 4)) || (o_rs | o_hs | w_rs | w_hs) % 8 != 0)
    return fail(SWAMLA_ERR_MISALIGNED,
                "mla_merge_project: o_lat and w need 16-byte aligned bases and strides that are multiples of 8");
  swamla::MergeProjectArgs a{o_part, lse_part, o_lat, o_rs, o_hs, ad, cache_batch, cache_seq, n_rows,
                             n_splits, min_chunk, plan, R, w, w_rs, w_hs, y, y_rs, y_hs};
  a.H = H;
  const int rc = swamla::launch_merge_project(a, static_cast<hipStream_t>(stream));
  if (rc != 0) return hip_fail("mla_merge_project");
  return ok();
}

int mla_head_product(const void* x, int64_t x_rs, int64_t x_hs, const void* w, int64_t w_rs, int64_t w_hs,
                     void* y, int64_t y_rs, int64_t y_hs, int32_t M, int32_t N, int32_t K, int32_t H,
                     int32_t dtype, void* stream) {
  const char* fn = "mla_head_product";
  if (dtype != SWAMLA_DTYPE_BF16) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: dtype %d not built (bf16 only)", fn, dtype);
  if (M < 0 || N < 0 || H < 0 || H > 65535)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: M=%d N=%d H=%d out of range", fn, M, N, H);
  if (K < 64 || K > 512 || K % 64 != 0)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: K=%d (built: multiples of 64 up to 512)", fn, K);
  if (N % 4 != 0) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: N=%d is not a multiple of 4", fn, N);
  if (M == 0 || N == 0 || H == 0) return ok();
  if (!x || !w || !y) return fail(SWAMLA_ERR_INVALID_ARG, "%s: null x / w / y", fn);
  if (x_rs < 0 || x_hs < 0 || w_hs < 0 || y_rs < 0 || y_hs < 0 || w_rs < K)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: negative strides, or a w row stride below K", fn);
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 8) || (x_rs | x_hs | w_rs | w_hs) % 8 != 0 ||
      (y_rs | y_hs) % 4 != 0)
    return fail(SWAMLA_ERR_MISALIGNED, "%s: x and w need 16-byte aligned bases and strides that are multiples of "
                "8, y an 8-byte aligned base and strides that are multiples of 4", fn);
  int dev = 0, n_cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cus < 1)
    return hip_fail(fn);
  swamla::HeadProductArgs a{x, x_rs, x_hs, w, w_rs, w_hs, y, y_rs, y_hs, M, N, K};
  const int rc = swamla::launch_head_product(a, H, n_cus, static_cast<hipStream_t>(stream));
  if (rc == -1) return fail(SWAMLA_ERR_UNSUPPORTED, "%s: no kernel for K=%d", fn, K);
  if (rc != 0) return hip_fail(fn);
  return ok();
}

// ---- host-side test hooks: the kernels' bit-level conversions run on the CPU.
void mla_host_f32_to_e4m3(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = swamla::f32_to_e4m3(x[i]);
}
void mla_host_e4m3_to_f32(const uint8_t* c, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = swamla::e4m3_to_f32(c[i]);
}
void mla_host_e4m3x4_to_bf16(const uint32_t* w, uint16_t* out, int64_t n_words) {
  for (int64_t i = 0; i < n_words; ++i) {
    uint32_t lo, hi;
    swamla::e4m3x4_to_bf16x4(w[i], lo, hi);
    out[4 * i + 0] = lo & 0xFFFF;
    out[4 * i + 1] = lo >> 16;
    out[4 * i + 2] = hi & 0xFFFF;
    out[4 * i + 3] = hi >> 16;
  }
}
void mla_host_f32_to_bf16(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = swamla::f32_to_bf16(x[i]);
}

int mla_probe_read(const void* src, int64_t bytes, uint32_t* sink, int32_t grid, void* stream) {
  if (!src || !sink || bytes < 0 || bytes % 16 != 0 || grid < 1 || grid > 65535)
    return fail(SWAMLA_ERR_INVALID_ARG, "mla_probe_read: bad arguments (bytes=%lld, grid=%d)", (long long)bytes, grid);
  if (!aligned(src, 16) || !aligned(sink, 4))
    return fail(SWAMLA_ERR_MISALIGNED, "mla_probe_read: src must be 16-byte aligned, sink 4-byte");
  if (swamla::launch_read_probe(src, bytes / 16, sink, grid, static_cast<hipStream_t>(stream)) != 0)
    return hip_fail("mla_probe_read");
  return ok();
}

int mla_probe_cache_stream(const void* ckv_cache, const void* kpe_cache, const float* ckv_scale,
                           int64_t cache_batch, int64_t cache_seq, const int32_t* start_pos, int32_t n_rows,
                           int32_t R, int32_t n_splits, int32_t min_chunk, int32_t cache_dtype, uint32_t* sink,
                           void* stream) {
  const char* fn = "mla_probe_cache_stream";
  if (int e = check_geometry(16, R, 64)) return e;
  if (swamla::padded_rank(R) > 64 * swamla::kMaxNB)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: kv_lora_rank %d (built up to %d)", fn, R, 64 * swamla::kMaxNB);
  if (cache_dtype != SWAMLA_DTYPE_BF16 && cache_dtype != SWAMLA_DTYPE_FP8)
    return fail(SWAMLA_ERR_UNSUPPORTED, "%s: cache dtype %d (bf16 or fp8 caches of a bf16 model)", fn, cache_dtype);
  if (!ckv_cache || !kpe_cache || !start_pos || !sink || (cache_dtype == SWAMLA_DTYPE_FP8 && !ckv_scale))
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: null pointer", fn);
  if (n_rows < 0 || n_rows > 65535 || n_splits < 1 || n_splits > 1024 || min_chunk < 1 || cache_batch < 1 ||
      cache_seq < 1 || cache_seq > (int64_t(1) << 31) - 1)
    return fail(SWAMLA_ERR_INVALID_ARG, "%s: bad arguments (n_rows=%d, n_splits=%d, min_chunk=%d)", fn, n_rows,
                n_splits, min_chunk);
  if (!aligned(ckv_cache, 16) || !aligned(kpe_cache, 16) || !aligned(sink, 4) ||
      (ckv_scale && !aligned(ckv_scale, 4)))
    return fail(SWAMLA_ERR_MISALIGNED, "%s: caches must be 16-byte aligned", fn);
  swamla::DecodeArgs a{};
  a.R = R;
  a.ckv = ckv_cache;
  a.kpe = kpe_cache;
  a.ckv_scale = ckv_scale;
  a.cache_b = cache_batch;
  a.cache_s = cache_seq;
  a.ad = swamla::Addressing{nullptr, nullptr, nullptr, start_pos, 1, 0};
  a.n_rows = n_rows;
  a.n_splits = n_splits;
  a.min_chunk = min_chunk;
  if (swamla::launch_stream_probe(a, cache_dtype, sink, static_cast<hipStream_t>(stream)) != 0)
    return hip_fail(fn);
  return ok();
}

}  // extern "C"
