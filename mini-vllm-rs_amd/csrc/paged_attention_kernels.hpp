// Internal launch interface between the C ABI (mvr_attn_api.cpp) and the
// HIP kernels (paged_attention.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvr {

// Tokens per MFMA chunk: one 16x16 tile of the score matrix per chunk.
constexpr int kChunkTokens = 16;
constexpr int kWaveSize = 64;
constexpr int kWavesPerBlock = 4;

// Head dimensions.  64 and 128 (every model shape the reference runs) take
// every plan: block merge, dense, deep pipeline, token pages and the
// chunked-prefill kernel.  The other multiples of 32 up to 256 take the
// split-context kernel with 16-row tiles in 1-wavefront blocks and the merge
// pass, for every call shape (page sizes that are not a multiple of 16 are
// repacked first).
constexpr bool head_dim_supported(int d) { return d >= 32 && d <= 256 && d % 32 == 0; }
constexpr bool head_dim_all_plans(int d) { return d == 64 || d == 128; }

// Token pages (page sizes that are not a multiple of 16, read in place) keep
// the element offsets within a page of all KV heads in 32 bits: such a page
// must hold fewer than 2^31 elements (larger ones are repacked).
constexpr bool token_page_offsets_fit(int num_kv_heads, int page_size, int head_dim) {
  return (long long)num_kv_heads * page_size * head_dim < (1LL << 31);
}

// One launch of the split-context kernel.  A "unit" is the work of one
// wavefront: (sequence b, kv head h, row tile rt, context partition part).
// Rows of a kv head are the grouped query rows rho = r*q_len + i (r = query
// head within the group, i = query position), the order of the reference's
// grouped matmul (common.rs:846-858).
struct PagedAttentionParams {
  const void* q;
  int64_t q_stride_head, q_stride_token;
  const void* key_pool;
  const void* value_pool;
  const int32_t* block_tables;
  int32_t block_table_stride;
  const int32_t* seq_lens;  // may be null: single_seq_len
  const int32_t* cu_q_lens; // may be null: single_q_len
  int32_t single_seq_len, single_q_len;
  void* out;
  int64_t out_stride_head, out_stride_token;
  float* partial_o;  // [units][row_tile_rows][head_dim] fp32, unnormalised
  float* partial_ml; // [units][row_tile_rows][2]: running max (log2 domain), sum
  int32_t num_seqs, num_kv_heads, group_size, page_size;
  int32_t chunks_per_part; // 16-token chunks per context partition
  int32_t max_parts;       // partitions per (sequence, kv head, row tile) in the grid
  int32_t row_tiles;       // row tiles per (sequence, kv head)
  int64_t num_units;
  float scale_log2; // softmax scale * log2(e)
  // Cascade passes (all optional, null / 0 otherwise):
  const int32_t* key_begin; // per sequence: first key (a multiple of 16); earlier keys belong to the prefix pass
  const int32_t* key_end;   // per sequence: prefix pass, keys [0, key_end), every query row sees all of them
  float* state_o;           // write normalised fp32 rows [q head][state_tokens][D] instead of `out` ...
  float* state_lse;         // ... and their log2-sum-exp [q head][state_tokens]
  int32_t state_tokens;
  // Cascade suffix pass (optional): before a row of `out` is written, it is
  // merged with the prefix pass's state of that row, for sequences whose
  // seq_prefix_len is > 0:  out = (2^(la-M) o_a + 2^(lb-M) o_b) / (2^(la-M) + 2^(lb-M)).
  const float* prefix_o;          // [q head][state_tokens][D], normalised
  const float* prefix_lse;        // [q head][state_tokens], log2 units
  const int32_t* seq_prefix_len;  // [num_seqs]
  // Sequences whose q_len lies outside [class_q_min, class_q_max] (0 = no
  // upper bound) belong to another launch of the same call and are skipped:
  // a batch mixing decode-sized and prefill-sized requests runs each class
  // on a grid planned for it.
  int32_t class_q_min, class_q_max;
  // Token pages (page sizes that are not a multiple of 16): page of token t =
  // t * page_magic >> page_magic_shift (mvr::page_divider).
  uint64_t page_magic;
  int32_t page_magic_shift;
};

// Grid shape chosen by the host.
struct PagedAttentionPlan {
  int dtype;      // 0 f32, 1 f16
  int head_dim;   // head_dim_supported()
  int row_blocks; // 16-row MFMA blocks per wavefront (1 or 2)
  int row_tiles;
  int chunks_per_part;
  int max_parts;
  int64_t num_units;
  size_t partial_bytes; // workspace for partials (0 when max_parts == 1)
  bool prefill;         // chunked-prefill kernel (paged_prefill.hip) instead of the split-context one
  int kv_splits;        // prefill: key-range splits per 128-row tile
  int prefill_groups;   // prefill: wavefront groups of 4 per block (2, or 1)
  bool block_merge;     // one block per tile, its partitions merged in LDS
  int block_waves;      // block_merge: wavefronts per block, 4, 8 or 16 (>= max_parts)
  bool dense_parts;     // ragged split plan: live units first, in a dense order (see dense_unit)
  bool deep_pipeline;   // three chunks in flight per wavefront instead of two (16-row tiles only)
  int unit_waves;       // split plans without block merge: wavefronts per block, 1, 2 or 4 (0 means 4)
  bool token_pages;     // pages that do not hold whole 16-token chunks, read in place (page_size >= 2)
};

hipError_t launch_paged_attention(const PagedAttentionPlan& plan, PagedAttentionParams params, hipStream_t stream);


// Wavefronts of the plan's kernel variant the current device holds at once
// (occupancy x waves per block x CUs); 0 if the device cannot be queried.
int64_t paged_attention_resident_waves(int dtype, int head_dim, int row_blocks);

} // namespace mvr
