/*
 * swamla_mi355x_testing.h — test and measurement hooks of
 * libswamla_mi355x.so, outside the drop-in boundary.  No reference
 * counterpart: the reference relies on torch's own casts and has no kernels.
 *
 *   mla_host_*   the kernels' bit-level conversions run on the CPU, so tests
 *                can pin the exact rounding the gfx950 code applies without
 *                a GPU;
 *   mla_probe_*  measurement kernels for bench.py's roofline ceiling: the
 *                plain HBM read rate, and a decode launch's cache stream with
 *                no arithmetic.  The module never calls them.
 */
#ifndef SWAMLA_MI355X_TESTING_H
#define SWAMLA_MI355X_TESTING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 -> e4m3fn codes, RNE, NaN for |x| > 464 (the append kernel's encoder). */
void mla_host_f32_to_e4m3(const float* x, uint8_t* out, int64_t n);
/* e4m3fn codes -> fp32 (exact). */
void mla_host_e4m3_to_f32(const uint8_t* c, float* out, int64_t n);
/* packed 4 x e4m3 words -> 4 x bf16 each (the decode kernel's dequantiser). */
void mla_host_e4m3x4_to_bf16(const uint32_t* w, uint16_t* out, int64_t n_words);
/* fp32 -> bf16 RNE (eager PyTorch's per-op rounding). */
void mla_host_f32_to_bf16(const float* x, uint16_t* out, int64_t n);

/* Reads `bytes` (a multiple of 16, 16-byte aligned `src`) once with 16-byte
 * non-temporal loads from `grid` workgroups of 256 threads and stores one
 * checksum word per thread in sink[grid * 256]. */
int mla_probe_read(const void* src, int64_t bytes, uint32_t* sink, int32_t grid, void* stream);

/* The cache stream of mla_decode_attn's bf16-model launch over `n_rows` dense
 * rows (row r attends [0, start_pos[r] + 1), as with rows_per_seq = 1), with
 * the static split plan (n_splits, min_chunk): the same grid, LDS ring, DMA
 * instructions and waits, no arithmetic.  Stores one checksum word per thread
 * in sink[n_splits * n_rows * 256]. */
int mla_probe_cache_stream(const void* ckv_cache, const void* kpe_cache, const float* ckv_scale,
                           int64_t cache_batch, int64_t cache_seq, const int32_t* start_pos, int32_t n_rows,
                           int32_t R, int32_t n_splits, int32_t min_chunk, int32_t cache_dtype, uint32_t* sink,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SWAMLA_MI355X_TESTING_H */
