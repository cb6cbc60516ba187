// mla_args.h — kernel argument blocks shared by the kernels and the C-ABI
// layer (plain pointers and sizes; passed to the kernels by value).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace swamla {

constexpr int kMaxNB = 8;  // latent rows of at most 64 kMaxNB = 512 channels for the MFMA kernels
// Ranks up to 64 kMaxNBWide = 1024 channels: the append, the merge and the
// wide-rank decode kernel (mla_decode_vec).
constexpr int kMaxNBWide = 16;

// Padded latent width of a rank: R_pad = 64 ceil(R / 64).
inline constexpr int padded_rank(int R) { return 64 * ((R + 63) / 64); }

// Where token / query-row positions come from.  Explicit mode: per-entry
// arrays.  Dense mode (start_pos != nullptr): entry i belongs to sequence
// i / T at position start_pos[i / T] + i % T, the layout of the reference's
// forward (x[B, T, dim] at one start position per sequence).
struct Addressing {
  const int32_t* seq;        // explicit: cache row of each entry
  const int32_t* pos;        // explicit append: destination position; decode: kv_len
  const int32_t* rope;       // explicit: RoPE table row
  const int32_t* start_pos;  // dense: [n / T] first position of each sequence
  int32_t T;                 // dense: entries per sequence
  int32_t rope_abs;          // dense: RoPE row = position (1) or t = i % T (0)
};

struct AppendArgs {
  const void* kv_in;  // rows [R_pad latent | P rope]
  int64_t in_rs;
  int n_tok;
  int R;  // kv_lora_rank; rows are R_pad = 64 ceil(R / 64) channels
  Addressing ad;
  const void* ln_w;
  const void* ln_b;
  float eps;
  const void* cos_tab;
  const void* sin_tab;
  int64_t rope_len;
  void* ckv;
  void* kpe;
  float* ckv_scale;
  int64_t cache_b;
  int64_t cache_s;
  int32_t* err_flag;
};

struct DecodeArgs {
  int R;  // kv_lora_rank; latent rows (cache, queries, outputs) are R_pad = 64 ceil(R / 64) channels
  const void* q_abs;
  int64_t qa_rs, qa_hs;
  const void* q_pe;
  int64_t qp_rs, qp_hs;
  const void* cos_tab;
  const void* sin_tab;
  int64_t rope_len;
  const void* ckv;
  const void* kpe;
  const float* ckv_scale;
  int64_t cache_b, cache_s;
  Addressing ad;  // pos = kv_len in explicit mode
  int n_rows;
  float scale_log2;  // softmax_scale * log2(e)
  int n_splits, min_chunk;
  // Length-balanced plan (balance > 0: a one-dimensional grid of `balance`
  // workgroups, the chunk chosen on the device and written to *plan).
  int balance;
  int32_t* plan;
  float* o_part;
  float* lse_part;
  void* o_lat;
  int64_t o_rs, o_hs;
  float* lse_out;  // optional [rows, H]: log-sum-exp of the rows finished in this launch (one split)
  // Optional fused append of one new token per row (fa.kv_in == nullptr:
  // none): the block owning a row's last split appends row r's token r.
  // fa.ad is always this launch's `ad` (dense, T = 1): the kernel derives the
  // token's position from the row's.
  AppendArgs fa;
  int H = 16;  // query heads: 16, or 32 (bf16 model and cache: one launch of two head groups)
};

struct MergeArgs {
  const float* o_part;
  const float* lse_part;
  Addressing ad;  // row lengths, clamped to the cache as the decode kernel does
  int64_t cache_b, cache_s;
  int n_rows, n_splits, min_chunk;
  const int32_t* plan;  // balanced plan: the chunk the decode launch chose (else null)
  int R;                // kv_lora_rank (rows of R_pad channels)
  void* o_lat;
  int64_t o_rs, o_hs;
  float* lse_out;
  int H = 16;  // heads of the partials ([rows, splits, H, R_pad]) and outputs
};

// Batched small-row linear layer: Y[b] = X[b] W[b]^T (+ bias[b]), bf16.
// Element strides: rows (_rs) and batch entries (_bs); columns are unit-stride.
struct LinearArgs {
  const void* x;
  int64_t x_rs, x_bs;
  const void* w;
  int64_t w_rs, w_bs;
  const void* bias;
  int64_t bias_bs;
  void* y;
  int64_t y_rs, y_bs;
  int M, N, K;
};

// Split merge fused with the per-head W_uv product: y[r, h, :] =
// W_uv[h] . merge_s(o_part[r, s, h, :]) (or o_lat[r, h, :] for one split).
struct MergeProjectArgs {
  const float* o_part;
  const float* lse_part;
  const void* o_lat;
  int64_t ol_rs, ol_hs;
  Addressing ad;  // row lengths, clamped to the cache as the decode kernel does
  int64_t cache_b, cache_s;
  int n_rows, n_splits, min_chunk;
  const int32_t* plan;  // balanced plan: the chunk the decode launch chose (else null)
  int R;                // kv_lora_rank (rows of R_pad channels)
  const void* w;
  int64_t w_rs, w_hs;
  void* y;
  int64_t y_rs, y_hs;
  int H = 16;  // heads of the partials ([rows, splits, H, R_pad]) and of y
};

int launch_append(const AppendArgs& a, int in_dt, int c_dt, hipStream_t s);
int launch_decode(const DecodeArgs& a, int dt, int c_dt, hipStream_t s);
// Workgroups of the decode launch one CU holds at once (HIP occupancy of the
// instance launch_decode picks); -1 for a combination without a kernel, -2
// when the HIP query fails.
int decode_blocks_per_cu(int dt, int c_dt, int R, bool fuse, int* blocks);
int launch_merge(const MergeArgs& a, int dt, hipStream_t s);
int launch_prefill(const DecodeArgs& a, int dt, int c_dt, hipStream_t s);
// Product with a packed weight (see mla_pack_weight): Y = X . W^T (+ bias).
struct PackedLinearArgs {
  const void* x;
  int64_t x_rs;
  const void* wp;  // packed W
  const void* bias;
  void* y;
  int64_t y_rs;
  int M, N, K;
  // Optional: adv[0 .. n_adv) += 1 (a decode loop's device positions, advanced
  // by the step's last launch instead of a kernel of its own; nothing in the
  // product reads them).  n_adv <= the workgroup's 512 threads.
  int32_t* adv;
  int n_adv;
};

struct PackWeightArgs {
  const void* w;
  int64_t w_rs;
  void* wp;
  int N, K;
};

// Per-head product of the prompt pass: y[m, h, n] = sum_k x[m, h, k] w[h, n, k]
// (strides in elements; m < M, n < N, k < K).
struct HeadProductArgs {
  const void* x;
  int64_t x_rs, x_hs;
  const void* w;
  int64_t w_rs, w_hs;
  void* y;
  int64_t y_rs, y_hs;
  int M, N, K;
};

// Measurement kernels (bench.py's roofline ceiling legs): a decode launch's
// cache stream alone (static plan; sink: n_splits * n_rows * 256 words) and
// a plain non-temporal read of n16 16-byte words (sink: grid * 256 words).
int launch_stream_probe(const DecodeArgs& a, int c_dt, uint32_t* sink, hipStream_t s);
int launch_read_probe(const void* src, int64_t n16, uint32_t* sink, int grid, hipStream_t s);

int launch_linear(const LinearArgs& a, int batch, hipStream_t s);
int launch_linear_packed(const PackedLinearArgs& a, hipStream_t s);
int launch_pack_weight(const PackWeightArgs& a, hipStream_t s);
int launch_merge_project(const MergeProjectArgs& a, hipStream_t s);
// -1: no kernel for this K; -2: launch error.
int launch_head_product(const HeadProductArgs& a, int H, int n_cus, hipStream_t s);

}  // namespace swamla
