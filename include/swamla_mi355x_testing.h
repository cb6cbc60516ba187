/*
 * swamla_mi355x_testing.h — host-side hooks of libswamla_mi355x.so that run
 * the kernels' bit-level conversions on the CPU.  They exist so tests can pin
 * the exact rounding the gfx950 code applies without a GPU.  No reference
 * counterpart: the reference relies on torch's own casts.
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

#ifdef __cplusplus
}
#endif

#endif /* SWAMLA_MI355X_TESTING_H */
