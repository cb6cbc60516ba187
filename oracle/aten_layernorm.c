/* aten_layernorm.c — TEST INFRASTRUCTURE ONLY (oracle; never linked into the
 * product library).
 *
 * CPU restatement of the LayerNorm that the reference's cache path calls:
 * `self.kv_norm(kv)` (models/mla.py:107 builds `nn.LayerNorm(kv_lora_rank)`,
 * :409 applies it) executed by PyTorch's CPU kernel.  The arithmetic lives in
 * the third-party dependency PyTorch (requirements.txt:2, torch >= 2.10.0;
 * this image: 2.10.0+rocm7.0, built with GCC 11.2), not in /root/reference.
 * Its published structure — a vectorised Welford moments pass followed by a
 * per-element affine — is restated here op by op, every product and sum
 * rounded where the compiled kernel rounds it (fused multiply-adds spelled
 * out with fmaf, everything else under -ffp-contract=off):
 *
 *   moments (one row of N values, converted to fp32):
 *     input vectors of V values (V = 16 for bf16 input, 8 for fp32), each
 *     seen as V/8 float vectors of 8 lanes ("halves");
 *     n = N / V vectors, cut into chunks of 16 vectors; per chunk, per half,
 *     per lane k a Welford stream over the chunk's vectors j = 0..:
 *         d = x - m1;  m1 = fma(d, fl(1/(j+1)), m1);  m2 = fma(d, x - m1, m2)
 *     each stream (count m0) is merged into a stack of 8-lane accumulators
 *     (a binary counter over the chunks, depth ceil(log2(chunks)), >= 1):
 *         c = fl(cnt_add / cnt_new);  dc = d * c;  m1 = m1 + dc;
 *         m2 = fma(dc, d * fl(cnt_old), m2 + m2_add)
 *     then the N - nV tail values go through a scalar Welford
 *         d = x - m1;  m1 = m1 + d / cnt;  m2 = fma(d, x - m1, m2)
 *     and the 8 lanes are merged into it one by one, each carrying n V / 8:
 *         c = fl(cnt_add / cnt_new);  m1 = fma(d, c, m1);
 *         m2 = m2 + fma((d * d) * c, fl(cnt_old), m2_add)
 *     var = m2 / N (biased);  rstd = 1 / sqrt(var + eps)   (fp32 throughout)
 *   affine:
 *     bf16 input:  y = fma(fma(x, rstd, -rstd * mean), w, b)
 *     fp32 input:  y = fma((x - mean) * rstd, w, b)
 *   and the bf16 result is rounded to nearest-even.
 *
 * How this is pinned (tests/test_oracle.py): bit-for-bit against
 * torch.nn.functional.layer_norm / torch.native_layer_norm (outputs, means
 * and rstds) on CPU over every rank 1..512 the kernels support, bf16 and fp32,
 * unit and random affine parameters, and row families from tiny to heavy
 * tailed and large-offset; `variant` plants single-site changes (a fused
 * multiply-add split, the stack merge reordered) that those comparisons must
 * reject.  The comparison is against the library routine the reference calls,
 * so it holds for the x86-64 hosts torch runs its AVX2 kernel on (AVX2 and
 * AVX-512 machines alike); the GPU tests repeat it on the GPU box's host.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define LANES 8
#define CHUNK 16
#define MAX_DEPTH 8

/* variant bits (planted mistakes for the tests; 0 = the statement above) */
#define V_SPLIT_WELFORD_FMA 1 /* Welford m1 update as m1 + d*c */
#define V_FUSE_STACK_M1 2     /* stack merge m1 update as fma(d, c, m1) */
#define V_LANE_M2_ORDER 4     /* lane merge m2 as fma(..., m2 + m2_add) */
#define V_SPLIT_AFFINE 8      /* affine without fused multiply-adds */

typedef struct {
  int64_t cnt;
  float m1[LANES], m2[LANES];
} acc8;

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static int ceil_log2_min1(int64_t x) {
  if (x <= 2) return 1;
  int r = 0;
  for (int64_t t = x - 1; t; t >>= 1) ++r;
  return r;
}

/* merge (cnt_add, a1, a2) into the 8-lane accumulator s */
static void stack_merge(int64_t cnt_add, const float* a1, const float* a2, acc8* s, int variant) {
  const int64_t cnt = s->cnt + cnt_add;
  const float c = cnt == 0 ? 0.f : (float)cnt_add / (float)cnt;
  const float old = (float)s->cnt;
  for (int k = 0; k < LANES; ++k) {
    const float d = a1[k] - s->m1[k];
    const float dc = d * c;
    s->m1[k] = (variant & V_FUSE_STACK_M1) ? fmaf(d, c, s->m1[k]) : s->m1[k] + dc;
    s->m2[k] = fmaf(dc, d * old, s->m2[k] + a2[k]);
  }
  s->cnt = cnt;
}

/* mean and biased variance of x[0..N) (fp32 values), V values per input vector */
static void welford_moments(const float* x, int N, int V, int variant, float* mean, float* var) {
  const int halves = V / LANES;
  const int64_t n = N / V;
  const int64_t chunks = (n + CHUNK - 1) / CHUNK;
  const int depth = ceil_log2_min1(chunks);
  acc8 stk[MAX_DEPTH];
  memset(stk, 0, sizeof(stk));
  for (int64_t i = 0; i < chunks; ++i) {
    const float* X = x + i * CHUNK * V;
    const int64_t cnt = n - i * CHUNK < CHUNK ? n - i * CHUNK : CHUNK;
    for (int h = 0; h < halves; ++h) {
      float a1[LANES], a2[LANES];
      for (int k = 0; k < LANES; ++k) {
        float m1 = 0.f, m2 = 0.f;
        for (int64_t j = 0; j < cnt; ++j) {
          const float xv = X[j * V + LANES * h + k];
          const float c = 1.0f / (float)(j + 1);
          const float d = xv - m1;
          m1 = (variant & V_SPLIT_WELFORD_FMA) ? m1 + d * c : fmaf(d, c, m1);
          m2 = fmaf(d, xv - m1, m2);
        }
        a1[k] = m1;
        a2[k] = m2;
      }
      stack_merge(cnt, a1, a2, &stk[0], variant);
    }
    int64_t carry = i + 1;
    for (int j = 1; j < depth && (carry & 1) == 0; ++j) {
      stack_merge(stk[j - 1].cnt, stk[j - 1].m1, stk[j - 1].m2, &stk[j], variant);
      memset(&stk[j - 1], 0, sizeof(acc8));
      carry >>= 1;
    }
  }
  for (int j = 1; j < depth; ++j) stack_merge(stk[j].cnt, stk[j].m1, stk[j].m2, &stk[0], variant);

  int64_t cnt = 0;
  float m1 = 0.f, m2 = 0.f;
  for (int64_t i = n * V; i < N; ++i) {
    const float xv = x[i];
    const float d = xv - m1;
    ++cnt;
    m1 = m1 + d / (float)cnt;
    m2 = fmaf(d, xv - m1, m2);
  }
  const int64_t per_lane = n * V / LANES;
  for (int k = 0; k < LANES; ++k) {
    const int64_t tot = cnt + per_lane;
    const float c = tot == 0 ? 0.f : (float)per_lane / (float)tot;
    const float d = stk[0].m1[k] - m1;
    m1 = fmaf(d, c, m1);
    const float t = (d * d) * c;
    if (variant & V_LANE_M2_ORDER)
      m2 = fmaf(t, (float)cnt, m2 + stk[0].m2[k]);
    else
      m2 = m2 + fmaf(t, (float)cnt, stk[0].m2[k]);
    cnt = tot;
  }
  *mean = m1;
  *var = m2 / (float)N;
}

/* bf16 rows x [M, N] (row stride x_rs elements) -> y (row stride y_rs);
 * w, b: N bf16 affine parameters; mean / rstd (may be NULL): per-row fp32. */
void aten_layernorm_bf16(const uint16_t* x, int64_t x_rs, int M, int N, const uint16_t* w, const uint16_t* b,
                         float eps, uint16_t* y, int64_t y_rs, float* mean_out, float* rstd_out, int variant) {
  float buf[4096];
  if (N > 4096) return;
  for (int r = 0; r < M; ++r) {
    const uint16_t* xr = x + (int64_t)r * x_rs;
    for (int i = 0; i < N; ++i) buf[i] = bf16_to_f32(xr[i]);
    float mean, var;
    welford_moments(buf, N, 16, variant, &mean, &var);
    const float rstd = 1.0f / sqrtf(var + eps);
    const float bias = -rstd * mean;
    if (mean_out) mean_out[r] = mean;
    if (rstd_out) rstd_out[r] = rstd;
    uint16_t* yr = y + (int64_t)r * y_rs;
    for (int i = 0; i < N; ++i) {
      const float g = bf16_to_f32(w[i]), be = bf16_to_f32(b[i]);
      const float o = (variant & V_SPLIT_AFFINE) ? (buf[i] * rstd + bias) * g + be
                                                 : fmaf(fmaf(buf[i], rstd, bias), g, be);
      yr[i] = f32_to_bf16_rne(o);
    }
  }
}

void aten_layernorm_f32(const float* x, int64_t x_rs, int M, int N, const float* w, const float* b, float eps,
                        float* y, int64_t y_rs, float* mean_out, float* rstd_out, int variant) {
  for (int r = 0; r < M; ++r) {
    const float* xr = x + (int64_t)r * x_rs;
    float mean, var;
    welford_moments(xr, N, 8, variant, &mean, &var);
    const float rstd = 1.0f / sqrtf(var + eps);
    if (mean_out) mean_out[r] = mean;
    if (rstd_out) rstd_out[r] = rstd;
    float* yr = y + (int64_t)r * y_rs;
    for (int i = 0; i < N; ++i) {
      const float t = (xr[i] - mean) * rstd;
      yr[i] = (variant & V_SPLIT_AFFINE) ? t * w[i] + b[i] : fmaf(t, w[i], b[i]);
    }
  }
}
