// mla_args.h — kernel argument blocks shared by the kernels and the C-ABI
// layer (plain pointers and sizes; passed to the kernels by value).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace swamla {

struct AppendArgs {
  const void* kv_in;
  int64_t in_rs;
  int n_tok;
  const int32_t* seq_idx;
  const int32_t* dst_pos;
  const int32_t* rope_pos;
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
  const void* q_abs;
  int64_t qa_rs, qa_hs;
  const void* q_pe;
  int64_t qp_rs, qp_hs;
  const int32_t* q_rope_pos;
  const void* cos_tab;
  const void* sin_tab;
  int64_t rope_len;
  const void* ckv;
  const void* kpe;
  const float* ckv_scale;
  int64_t cache_b, cache_s;
  const int32_t* row_seq;
  const int32_t* kv_len;
  int n_rows;
  float scale_log2;  // softmax_scale * log2(e)
  int n_splits, min_chunk;
  float* o_part;
  float* lse_part;
  void* o_lat;
  int64_t o_rs, o_hs;
};

struct MergeArgs {
  const float* o_part;
  const float* lse_part;
  const int32_t* kv_len;
  int n_rows, n_splits, min_chunk;
  void* o_lat;
  int64_t o_rs, o_hs;
  float* lse_out;
};

int launch_append(const AppendArgs& a, int in_dt, int c_dt, hipStream_t s);
int launch_decode(const DecodeArgs& a, int dt, int c_dt, hipStream_t s);
int launch_merge(const MergeArgs& a, int dt, hipStream_t s);

}  // namespace swamla
