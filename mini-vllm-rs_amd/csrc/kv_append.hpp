// Internal launch interface of the fused RoPE + KV-append kernel (kv_append.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvr {

struct RopeAppendParams {
  const void* q;
  int64_t q_stride_head, q_stride_token;
  const void* k;
  int64_t k_stride_head, k_stride_token;
  const void* v;
  int64_t v_stride_head, v_stride_token;
  const void* cos_table; // [rope_len, head_dim / 2]
  const void* sin_table;
  const int32_t* block_tables;
  int32_t block_table_stride;
  const int32_t* seq_lens;  // may be null: single_seq_len
  const int32_t* cu_q_lens; // may be null: single request of total_q tokens
  int32_t single_seq_len;
  void* q_out;
  int64_t q_out_stride_head, q_out_stride_token;
  void* key_pool;
  void* value_pool;
  int32_t num_seqs, num_q_heads, num_kv_heads, head_dim, page_size, total_q;
};

// dtype: 0 = F32, 1 = F16; rope_type: 0 = Neox, 1 = Interleaved.
hipError_t launch_rope_append(const RopeAppendParams& params, int dtype, int rope_type, hipStream_t stream);

} // namespace mvr
