/*
 * swamla_mi355x.h — C-ABI of the MI355X (gfx950) MLA latent-KV-cache kernels.
 *
 * Every entry point replaces one piece of the absorb branch of the reference
 * `MLA.forward` (Orolol/swamla, models/mla.py).  The library allocates no
 * memory and keeps no pointer after it returns; its only device state is the
 * fixed scratch area of mla_decode_attn_noalloc (one per GPU, part of the
 * loaded code object).  The caller owns caches, partial buffers and outputs.
 * Work is enqueued on the
 * caller's HIP stream (`stream` is a hipStream_t; NULL = default stream) and
 * nothing synchronises the host.  All entry points are graph-capturable.
 *
 * Return value: SWAMLA_OK (0) or a negative SWAMLA_ERR_* code; the message of
 * the last failure on the calling thread is returned by mla_last_error().
 *
 * Element types (the `*_dtype` arguments):
 *   SWAMLA_DTYPE_F32   IEEE binary32
 *   SWAMLA_DTYPE_BF16  bfloat16 (raw 16-bit storage)
 *   SWAMLA_DTYPE_FP8   OCP float8 e4m3fn with one fp32 scale per cached token
 *                      (latent c_kv only; k_pe stays in the model dtype)
 *
 * Geometry of this build: heads H = 16, qk_rope_head_dim P = 64 and any
 * kv_lora_rank 1 <= R <= 1024 (the real model scales the rank per layer,
 * models/swa_mla_model.py:216-247, up to twice its base).  mla_append,
 * mla_merge, mla_decode_attn and mla_decode_attn_noalloc take every such
 * rank (decode attention above 512 runs a channel-split MFMA kernel for a
 * bf16 model, bf16 or e4m3 cache, and a VALU kernel for fp32 models);
 * mla_decode_attn_append, mla_merge_project and the measurement probes take
 * R <= 512, mla_prefill_attn R <= 256.
 * mla_decode_attn, mla_decode_attn_append, mla_merge and mla_merge_project
 * also take H = 32 in one launch for a bf16 model with R_pad <= 256 (the
 * reference's xl preset, models/swa_mla_model.py:618-640: each decode wave
 * serves two 16-head groups from the same cache tiles, streamed once).
 * Other values return SWAMLA_ERR_UNSUPPORTED.  Latent rows are laid out with
 * R_pad = 64 * ceil(R / 64) channels (R_pad = R for the BASELINE rank 256):
 * caches, queries, outputs, partials and the latent half of input rows hold
 * R_pad values per token / head.  The kernels write zeros into channels
 * R .. R_pad-1 of cache rows and outputs and ignore those channels of their
 * inputs, except that a cache's padding must hold the zeros mla_append wrote
 * (a zero-filled allocation does).
 */
#ifndef SWAMLA_MI355X_H
#define SWAMLA_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SWAMLA_ABI_VERSION 6

enum {
  SWAMLA_OK = 0,
  SWAMLA_ERR_INVALID_ARG = -1,  /* null pointer, negative size, bad stride  */
  SWAMLA_ERR_UNSUPPORTED = -2,  /* geometry / dtype combination not built   */
  SWAMLA_ERR_MISALIGNED = -3,   /* pointer or stride breaks 16-byte loads   */
  SWAMLA_ERR_OUT_OF_RANGE = -4, /* position beyond the cache / rope table   */
  SWAMLA_ERR_HIP = -5           /* the HIP runtime rejected a launch        */
};

enum { SWAMLA_DTYPE_F32 = 0, SWAMLA_DTYPE_BF16 = 1, SWAMLA_DTYPE_FP8 = 2 };

/* ABI revision of the loaded library; callers compare it with
 * SWAMLA_ABI_VERSION.  No reference counterpart (the reference has no FFI). */
int mla_abi_version(void);

/* Message describing the last non-zero return on this thread ("" if none).
 * No reference counterpart: the reference raises Python exceptions. */
const char* mla_last_error(void);

/*
 * Addressing of tokens (mla_append) and query rows (mla_decode_attn,
 * mla_merge) — exactly one of two modes per call:
 *   explicit  per-entry int32 device arrays (cache row, position, RoPE row);
 *             start_pos must be NULL.
 *   dense     start_pos = int32 device array [n / T]: entry i belongs to cache
 *             row i / T at position start_pos[i / T] + i % T — the layout of
 *             the reference's forward(x[B, T, dim], start_pos) with one start
 *             position per sequence (mla.py:277-278, :413-418).  RoPE row is
 *             i % T when rope_abs = 0 (the reference's chunk-local positions,
 *             positional_encoding.py:49-50) or the absolute position when 1.
 *             The per-entry arrays must be NULL.
 */

/*
 * mla_append — fused cache append (one call per forward, any T).
 * Replaces models/mla.py:307-323 (split of wkv_a(x) into c / k_pe and RoPE on
 * k_pe), :409 (kv_norm LayerNorm) and :413-414 (scatter into kv_cache /
 * pe_cache at [:bsz, start_pos:end_pos]).
 *
 * kv_in        [n_tok, in_row_stride] rows in in_dtype; columns 0..R-1 are the
 *              latent c (R..R_pad-1 ignored), R_pad..R_pad+P-1 are k_pe (for
 *              R = R_pad the wkv_a output itself, no copy needed).
 * seq_idx, dst_pos, rope_pos   explicit addressing: cache row, cache position
 *              and RoPE table row of each token.
 * start_pos, tokens_per_seq, rope_abs   dense addressing (see above).
 * ln_w, ln_b   [R_pad] LayerNorm affine parameters in in_dtype (entries
 *              R.. ignored); eps as in torch.
 * cos_tab,     [rope_len, P/2] in in_dtype: the first P/2 columns of the
 * sin_tab      reference cos_cached / sin_cached (positional_encoding.py:21-28).
 * ckv_cache    [cache_batch, cache_seq, R_pad] in cache_dtype (u8 codes for
 *              FP8); the LayerNorm covers the R channels, R.. are written 0.
 * kpe_cache    [cache_batch, cache_seq, P] in in_dtype.
 * ckv_scale    [cache_batch, cache_seq] fp32, written only for FP8 (else NULL).
 * err_flag     optional device int32; a token whose cache row / position /
 *              RoPE row lies outside the buffers is skipped and sets it to 1.
 *
 * Numerics: the LayerNorm is PyTorch's CPU LayerNorm op for op (fp32 Welford
 * statistics in ATen's vectorised order, fused multiply-adds where its
 * compiled kernel fuses), so the latent rows equal the reference's
 * kv_norm(kv) bit for bit for bf16 and fp32 rows.
 * RoPE rounds after every multiply and add in in_dtype, as eager PyTorch does.
 * FP8: scale = max(amax, 1e-12) / 448 in fp32, code = RNE(y / scale).
 */
int mla_append(const void* kv_in, int64_t in_row_stride, int32_t n_tok,
               const int32_t* seq_idx, const int32_t* dst_pos,
               const int32_t* rope_pos, const int32_t* start_pos,
               int32_t tokens_per_seq, int32_t rope_abs, const void* ln_w,
               const void* ln_b, float eps, const void* cos_tab,
               const void* sin_tab, int64_t rope_len, void* ckv_cache,
               void* kpe_cache, float* ckv_scale, int64_t cache_batch,
               int64_t cache_seq, int32_t* err_flag, int32_t in_dtype,
               int32_t cache_dtype, int32_t R, int32_t P, void* stream);

/*
 * mla_decode_attn — absorbed attention of query rows over the latent cache.
 * Replaces models/mla.py:417-487 (cache gather, wkv_b up-projection of the
 * whole cache, cat with k_pe, SDPA with scale softmax_scale) by the
 * re-associated form  s_t = scale * (q_abs . c_t + rope(q_pe) . k_pe_t),
 * o_lat = sum_t softmax(s)_t c_t.
 *
 * Query row r attends to its cache row over positions [0, L): explicit mode
 * row_seq[r], L = kv_len[r], RoPE row q_rope_pos[r]; dense mode L = start +
 * r % T + 1 (causal, bottom-right for a prefill chunk).
 * q_abs        row r, head h at q_abs + r*q_abs_rs + h*q_abs_hs, R_pad values
 *              read (channels R.. ignored).
 * q_pe         row r, head h at q_pe + r*q_pe_rs + h*q_pe_hs, P values before
 *              RoPE; rotated in-kernel.
 * Split-KV: each row is cut into ns = ceil(L / chunk) splits of
 *   chunk = round_up(max(min_chunk, ceil(L / n_splits)), 16) tokens,
 * one workgroup each on a grid of n_splits x n_rows.
 * Balanced plan (balance_blocks > 0; for ragged batches): the launch is a
 * grid of balance_blocks workgroups and min_chunk is replaced by one chunk
 * c chosen on the device from all rows' lengths — the smallest multiple of
 * 64 tokens >= min_chunk with ceil(L_r / c) <= n_splits for every row and
 * sum_r max(1, ceil(L_r / c)) <= balance_blocks (mla_balanced_chunk
 * computes the same value on the host).  Row r gets ns_r =
 * ceil(ceil(L_r / 64) / (c / 64)) workgroups and is cut into near-equal
 * splits (the formula above with n_splits = ns_r and min_chunk = 1); the
 * workgroups take the rows' splits in row-major order.  c is written to
 * *plan (int32, may be NULL) for mla_merge / mla_merge_project.  Needs
 * n_rows <= balance_blocks, n_rows <= 256 and cache_seq <= 2^24.
 * Rows with ns == 1 are written straight to o_lat.  Others write normalised
 * partials o_part [n_rows, n_splits, H, R_pad] fp32 and log-sum-exp lse_part
 * [n_rows, n_splits, H] (natural log of sum exp(s)) that mla_merge combines.
 * o_lat        row r, head h at o_lat + r*o_rs + h*o_hs, R_pad values (R..
 *              written 0), in dtype.
 * lse_out      optional fp32 [n_rows, H] (may be NULL): the natural-log
 *              log-sum-exp of the scaled scores of every row this launch
 *              finishes (ns <= 1; -inf for an empty row); mla_merge writes the
 *              others'.
 */
int mla_decode_attn(const void* q_abs, int64_t q_abs_rs, int64_t q_abs_hs,
                    const void* q_pe, int64_t q_pe_rs, int64_t q_pe_hs,
                    const void* cos_tab, const void* sin_tab, int64_t rope_len,
                    const void* ckv_cache, const void* kpe_cache,
                    const float* ckv_scale, int64_t cache_batch,
                    int64_t cache_seq, const int32_t* row_seq,
                    const int32_t* kv_len, const int32_t* q_rope_pos,
                    const int32_t* start_pos, int32_t rows_per_seq,
                    int32_t rope_abs, int32_t n_rows, int32_t H, int32_t R,
                    int32_t P, float sm_scale, int32_t n_splits,
                    int32_t min_chunk, int32_t balance_blocks, int32_t* plan,
                    float* o_part, float* lse_part, void* o_lat, int64_t o_rs,
                    int64_t o_hs, float* lse_out, int32_t dtype,
                    int32_t cache_dtype, void* stream);

/*
 * mla_decode_attn_append — one decode step (one new token per sequence) with
 * the append folded into the attention launch.  Replaces, for T = 1,
 * models/mla.py:307-323 and :409-414 (mla_append's part) together with
 * :417-487 (mla_decode_attn's part).
 *
 * Dense addressing only, one query row per sequence: row r is cache row r,
 * its new token kv_in[r] is written at start_pos[r] exactly as mla_append
 * writes it (same LayerNorm / RoPE / e4m3 numerics), and row r then attends
 * over [0, start_pos[r] + 1) including that token, as mla_decode_attn does.
 * kv_in, in_row_stride, ln_w, ln_b, eps, err_flag: as for mla_append (bf16;
 * the k_pe RoPE uses cos_tab / sin_tab at the row's RoPE row).  The other
 * arguments are those of mla_decode_attn with row_seq / kv_len / q_rope_pos
 * absent and rows_per_seq = 1.  bf16 models only (bf16 or e4m3 cache).
 * A lane reads the R_pad / 64 channels it owns at once: kv_in, ln_w and
 * ln_b need bases aligned to A bytes, A the largest power of two from 4 to
 * 16 that divides 2 * (R_pad / 64) (4 if none does; 8 for R = 256), and
 * in_row_stride a multiple of A / 2 elements.
 * Results are identical to mla_append followed by mla_decode_attn.
 */
int mla_decode_attn_append(const void* kv_in, int64_t in_row_stride,
                           const void* ln_w, const void* ln_b, float eps,
                           int32_t* err_flag, const void* q_abs,
                           int64_t q_abs_rs, int64_t q_abs_hs,
                           const void* q_pe, int64_t q_pe_rs, int64_t q_pe_hs,
                           const void* cos_tab, const void* sin_tab,
                           int64_t rope_len, void* ckv_cache, void* kpe_cache,
                           float* ckv_scale, int64_t cache_batch,
                           int64_t cache_seq, const int32_t* start_pos,
                           int32_t rope_abs, int32_t n_rows, int32_t H,
                           int32_t R, int32_t P, float sm_scale,
                           int32_t n_splits, int32_t min_chunk,
                           int32_t balance_blocks, int32_t* plan, float* o_part,
                           float* lse_part, void* o_lat, int64_t o_rs,
                           int64_t o_hs, float* lse_out, int32_t dtype,
                           int32_t cache_dtype, void* stream);

/*
 * mla_decode_attn_noalloc — mla_decode_attn followed by mla_merge, with the
 * split partials, their log-sum-exps and the balanced plan kept in a fixed
 * scratch area inside the library instead of caller buffers.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc); it calls no allocating routine.
 * Arguments: those of mla_decode_attn without plan / o_part / lse_part;
 * o_lat and lse_out receive every row's merged result.  Limit: n_rows x
 * n_splits x H x R_pad x 4 bytes of partials at most 16 MiB (n_splits == 1
 * needs none); larger calls return SWAMLA_ERR_UNSUPPORTED.  There is one
 * scratch area per GPU (16.25 MiB of device memory on every GPU the library
 * loads on, held to the end of the process), shared by every call on it.
 * Calls on one stream are ordered by the stream; a call on another stream
 * is ordered after the device's last call (its stream waits for a completion
 * event the library records after each call; host threads take turns).
 * Calls under graph capture neither wait nor record: replays of graphs that
 * use the area on different streams race and must be ordered by the caller.  Nothing in the area needs clearing between calls
 * (each launch writes every partial it reads back).
 */
int mla_decode_attn_noalloc(const void* q_abs, int64_t q_abs_rs,
                            int64_t q_abs_hs, const void* q_pe,
                            int64_t q_pe_rs, int64_t q_pe_hs,
                            const void* cos_tab, const void* sin_tab,
                            int64_t rope_len, const void* ckv_cache,
                            const void* kpe_cache, const float* ckv_scale,
                            int64_t cache_batch, int64_t cache_seq,
                            const int32_t* row_seq, const int32_t* kv_len,
                            const int32_t* q_rope_pos,
                            const int32_t* start_pos, int32_t rows_per_seq,
                            int32_t rope_abs, int32_t n_rows, int32_t H,
                            int32_t R, int32_t P, float sm_scale,
                            int32_t n_splits, int32_t min_chunk,
                            int32_t balance_blocks, void* o_lat, int64_t o_rs,
                            int64_t o_hs, float* lse_out, int32_t dtype,
                            int32_t cache_dtype, void* stream);

/*
 * mla_prefill_attn — absorbed attention of a prefill chunk: T new query
 * tokens per sequence in dense addressing (row r = sequence r / T, token
 * t = r % T), each attending causally over positions [0, start_pos + t + 1)
 * of its cache row (bottom-right, as mla_decode_attn's dense mode).
 * Replaces models/mla.py:417-487 for seqlen > 1 (the reference aligns its
 * is_causal mask top-left, which differs only when start_pos > 0, :480-484).
 * Arguments as mla_decode_attn's dense mode (start_pos [n_rows / T],
 * tokens_per_seq = T, rope_abs), without split-KV: o_lat is written
 * directly.  One workgroup serves eight consecutive tokens of a sequence,
 * so each cache tile is read once per eight queries.  kv_lora_rank up to 256
 * (larger ranks: mla_decode_attn).  bf16 models only (bf16
 * or e4m3 cache).
 */
int mla_prefill_attn(const void* q_abs, int64_t q_abs_rs, int64_t q_abs_hs,
                     const void* q_pe, int64_t q_pe_rs, int64_t q_pe_hs,
                     const void* cos_tab, const void* sin_tab, int64_t rope_len,
                     const void* ckv_cache, const void* kpe_cache,
                     const float* ckv_scale, int64_t cache_batch,
                     int64_t cache_seq, const int32_t* start_pos,
                     int32_t tokens_per_seq, int32_t rope_abs, int32_t n_rows,
                     int32_t H, int32_t R, int32_t P, float sm_scale,
                     void* o_lat, int64_t o_rs, int64_t o_hs, int32_t dtype,
                     int32_t cache_dtype, void* stream);

/*
 * mla_merge — log-sum-exp merge of split-KV partials (no reference
 * counterpart: the reference attends in one SDPA call, mla.py:581-595).
 * o = sum_s exp(lse_s - M) o_s / sum_s exp(lse_s - M), M = max_s lse_s, for
 * every row whose split count (same formula as mla_decode_attn) exceeds 1.
 * Row lengths as mla_decode_attn derives them: row_seq / kv_len (explicit)
 * or start_pos / rows_per_seq (dense), clamped to cache_seq, 0 for a cache
 * row outside [0, cache_batch).  plan: the chunk a balanced mla_decode_attn
 * wrote (NULL when that launch used min_chunk).
 * lse_out [n_rows, H] fp32 is optional (NULL = not written).
 */
int mla_merge(const float* o_part, const float* lse_part,
              const int32_t* row_seq, const int32_t* kv_len,
              const int32_t* start_pos, int32_t rows_per_seq,
              int64_t cache_batch, int64_t cache_seq, int32_t n_rows,
              int32_t H, int32_t R, int32_t n_splits, int32_t min_chunk,
              const int32_t* plan, void* o_lat, int64_t o_rs, int64_t o_hs,
              float* lse_out, int32_t dtype, void* stream);

/*
 * mla_linear — batched linear layer for the few query rows of a decode step:
 *   y[b][m][n] = sum_k x[b][m][k] * w[b][n][k] (+ bias[b][n]),  b < batch,
 * bf16 inputs and output, fp32 accumulation, one rounding per output (what
 * a bf16 nn.Linear returns).  Replaces, for decode-sized inputs, the
 * step's GEMMs: wq (models/mla.py:281-288) and wkv_a (:307) as one product
 * over their stacked weights, the per-head absorbed products q_nope . W_uk
 * and o_lat . W_uv^T that re-associate the einsums of mla.py:427 and :433,
 * and wo (mla.py:490-495).
 * Element strides: x row x_rs / batch x_bs, w row w_rs / batch w_bs, y row
 * y_rs / batch y_bs, bias batch bias_bs; the k and n dimensions are
 * contiguous.  bias may be NULL.
 * Limits: 1 <= M <= 128, N a multiple of 16, K a multiple of 128, x and w
 * 16-byte aligned with row / batch strides that are multiples of 8.
 */
int mla_linear(const void* x, int64_t x_rs, int64_t x_bs, const void* w,
               int64_t w_rs, int64_t w_bs, const void* bias, int64_t bias_bs,
               void* y, int64_t y_rs, int64_t y_bs, int32_t M, int32_t N,
               int32_t K, int32_t batch, int32_t dtype, void* stream);

/*
 * mla_pack_weight — lays a [N, K] row-major weight out for
 * mla_linear_packed (no reference counterpart: a one-time re-layout of the
 * weights of wq / wkv_a (stacked) and wo, models/mla.py:281-288, :307,
 * :490-495).  Packed element (n, k) sits at
 *   (((n / 8) * (K / 64) + k / 64) * 8 + (k % 64) / 8) * 64 + (n % 8) * 8 + k % 8,
 * i.e. 1 KB tiles of 8 rows x 64 k, each read whole by one wavefront load.
 * w_packed holds N*K elements.  bf16; N a multiple of 8, K of 64; 16-byte
 * aligned bases, w_rs a multiple of 8 elements.
 */
int mla_pack_weight(const void* w, int64_t w_rs, int32_t N, int32_t K,
                    void* w_packed, int32_t dtype, void* stream);

/*
 * mla_linear_packed — y[m][n] = sum_k x[m][k] * w[n][k] (+ bias[n]) with w
 * packed by mla_pack_weight; bf16 in / out, fp32 accumulation, one rounding
 * per output.  Replaces the decode step's two large products: the stacked
 * wq / wkv_a product (models/mla.py:281-288, :307, with W_uk absorbed) and
 * wo (:490-495).
 * Limits: 0 <= M <= 128, N a multiple of 8, K in {512, 1024, 1536, 2048};
 * x and w_packed 16-byte aligned, x_rs a multiple of 8; y_rs >= N.
 * advance (optional, may be null): the launch also adds 1 to advance[0 ..
 * n_advance) (1 <= n_advance <= 512, 4-byte aligned, non-empty product).
 * No reference counterpart: the reference's MLA takes start_pos as a host
 * int (models/mla.py:232-236); a replayed HIP graph keeps the positions on
 * the device, and this lets a decode step's last product advance them
 * instead of a launch of its own.  The array must not overlap x, w_packed,
 * bias or y.
 */
int mla_linear_packed(const void* x, int64_t x_rs, const void* w_packed,
                      const void* bias, void* y, int64_t y_rs, int32_t M,
                      int32_t N, int32_t K, int32_t* advance,
                      int32_t n_advance, int32_t dtype, void* stream);

/*
 * mla_merge_project — split-KV merge fused with the W_uv read-out:
 *   y[r][h][d] = sum_c W_uv[h][d][c] * o_lat[r][h][c],
 * where o_lat is the log-sum-exp merge of the mla_decode_attn partials
 * (rows with more than one split, merged as mla_merge does and rounded to
 * bf16) or the o_lat row mla_decode_attn wrote itself (one split).
 * Replaces mla_merge followed by the per-head product with the value half of
 * wkv_b, i.e. the re-associated einsum of models/mla.py:433 and the reshape
 * to wo's input layout at :490-491.
 * Row lengths and splits are derived exactly as mla_decode_attn does (same
 * addressing arguments, same cache_batch / cache_seq clamping; plan as for
 * mla_merge).
 * w            head h, output d at w + h*w_hs + d*w_rs, R_pad values (for R =
 *              R_pad a view of wkv_b.weight: w_hs = (nope + Dv)*R, w_rs = R,
 *              base + nope*R; otherwise a zero-padded copy).
 * y            row r, head h at y + r*y_rs + h*y_hs, Dv values (wo's input
 *              [rows, H*Dv]: y_rs = H*Dv, y_hs = Dv).
 * o_part / lse_part may be NULL when n_splits == 1.  bf16 only, Dv = 128.
 */
int mla_merge_project(const float* o_part, const float* lse_part,
                      const void* o_lat, int64_t o_rs, int64_t o_hs,
                      const int32_t* kv_len, const int32_t* row_seq,
                      const int32_t* start_pos, int32_t rows_per_seq,
                      int64_t cache_batch, int64_t cache_seq, int32_t n_rows,
                      int32_t H, int32_t R, int32_t n_splits,
                      int32_t min_chunk, const int32_t* plan, const void* w,
                      int64_t w_rs, int64_t w_hs, int32_t Dv, void* y,
                      int64_t y_rs, int64_t y_hs, int32_t dtype, void* stream);

/*
 * mla_head_product — the per-head products of the prompt pass (prefill-side
 * absorption): y[m][h][n] = sum_k x[m][h][k] * w[h][n][k] for m < M, h < H,
 * n < N, k < K; bf16 in / out, fp32 accumulation, one round-to-nearest-even
 * rounding per output.  Replaces, for prompt-sized inputs, the einsums of
 * models/mla.py:427 and :433 in their re-associated (absorbed) form:
 *   q_abs = q_nope . W_uk   x = the wq output [M, H, 192] read in place,
 *                           w = W_uk^T [H, R_pad, 128], y = q_abs [M, H, R_pad];
 *   o = o_lat . W_uv^T      x = o_lat [M, H, R_pad], w = W_uv [H, 128, R_pad],
 *                           y = [M, H * 128], wo's input (mla.py:490-491).
 * Element strides: x row x_rs / head x_hs, w row (n) w_rs / head w_hs, y row
 * y_rs / head y_hs; k and n contiguous.
 * Limits: K a multiple of 64 up to 512, N a multiple of 4, H <= 65535; x and
 * w 16-byte aligned with strides that are multiples of 8, y 8-byte aligned
 * with strides that are multiples of 4.
 */
int mla_head_product(const void* x, int64_t x_rs, int64_t x_hs,
                     const void* w, int64_t w_rs, int64_t w_hs, void* y,
                     int64_t y_rs, int64_t y_hs, int32_t M, int32_t N,
                     int32_t K, int32_t H, int32_t dtype, void* stream);

/* Split plan used by both kernels, exported so hosts and tests can size the
 * partial buffers: number of splits of a row of length L (0 for L <= 0). */
int32_t mla_split_count(int32_t L, int32_t n_splits, int32_t min_chunk);

/* The chunk (tokens) of a balanced plan over host-side row lengths (already
 * clamped to the cache, at most 2^24; <= 0 for an empty row), as
 * mla_decode_attn chooses
 * it on the device; negative SWAMLA_ERR_* on bad arguments.  No reference
 * counterpart (the reference does not split the KV range). */
int32_t mla_balanced_chunk(const int32_t* lens, int32_t n_rows,
                           int32_t n_splits, int32_t min_chunk,
                           int32_t balance_blocks);

/* Decode workgroups per CU that the kernel mla_decode_attn (fused = 0) or
 * mla_decode_attn_append (fused = 1) launches for this dtype pair and rank
 * is built for, capped by the HIP occupancy of that kernel on the current
 * device: 1 for a bf16 cache and for fp32; 3 for an e4m3 cache at
 * R <= 256, whose kernel shares each CU among three workgroups to hide its
 * per-tile latency.  A
 * host sizes n_splits (static plan) or balance_blocks (balanced plan) for
 * CUs x this many workgroups.  Negative SWAMLA_ERR_* on an unsupported
 * combination or a failed HIP query.  No reference counterpart (the
 * reference does not split the KV range). */
int32_t mla_decode_blocks_per_cu(int32_t dtype, int32_t cache_dtype,
                                 int32_t R, int32_t fused);

#ifdef __cplusplus
}
#endif

#endif /* SWAMLA_MI355X_H */
