/*
 * ORACLE — test infrastructure only (see kv_append_oracle.c).
 * CPU restatement of the step before mini-vllm-rs's attention: rotary
 * embedding of the request's Q/K (src/models/backends/common.rs:294-307,
 * :344-359) and the append of K/V into the paged cache
 * (src/model_runner/server/kv_cache/paged_cache.rs:170-199, :290-327,
 * physical_page_pool.rs:188-209).  Never linked into the product.
 */
#ifndef MVR_KV_APPEND_ORACLE_H
#define MVR_KV_APPEND_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* RotaryEmbeddingType (common.rs:552-556): Neox rotates (i, i + D/2)
   (candle_nn::rotary_emb::rope), Interleaved rotates (2i, 2i + 1)
   (candle_nn::rotary_emb::rope_i); both use cos/sin[position][i]. */
enum { ORACLE_ROPE_NEOX = 0, ORACLE_ROPE_INTERLEAVED = 1 };

enum {
  ORACLE_APPEND_OK = 0,
  ORACLE_APPEND_E_INVALID = -1,
  ORACLE_APPEND_E_EMPTY = -2,     /* "cannot append an empty KV-cache tensor" (kv_cache/utils.rs:33-36) */
  ORACLE_APPEND_E_MISSING = -3,   /* the block table has no page for a position being written */
  ORACLE_APPEND_E_PAGE_ID = -4,   /* page id outside the pool */
  ORACLE_APPEND_E_READ_ONLY = -5, /* "cannot mutate written physical page N" (physical_page_pool.rs:197-201) */
  ORACLE_APPEND_E_ROPE_RANGE = -6 /* position beyond the cos/sin tables (Tensor::narrow fails) */
};

/* forward_rope for one request (common.rs:344-359) in the activation dtype
   (ORACLE_F32 / ORACLE_F16 of paged_attention_oracle.h).  x and y are
   [heads, q_len, head_dim] contiguous (y may alias x); cos_table/sin_table are
   [rope_len, head_dim/2] in the same dtype; token t uses row start_pos + t
   (cos.narrow(0, index_pos, query_len), common.rs:353-354). */
int oracle_rope(int dtype, int rope_type, const void* x, int heads, int q_len, int head_dim, const void* cos_table,
                const void* sin_table, int rope_len, int start_pos, void* y);

/* The same rotation in double precision with no rounding (independent check). */
int oracle_rope_f64(int rope_type, const double* x, int heads, int q_len, int head_dim, const double* cos_table,
                    const double* sin_table, int rope_len, int start_pos, double* y);

/* append_to_pages + PhysicalPagePool::write_page for one layer of one
   request: token_count tokens of key/value [num_kv_heads, token_count,
   head_dim] (elements of elem_size bytes, any dtype) go to positions
   cached_token_count .. cached_token_count + token_count - 1, position s in
   page page_ids[s / page_size], slot s % page_size.  page_ids is the layer's
   block table after the pages for this append were allocated.
   page_writable (one byte per pool page, nonzero = PendingWrite) may be NULL
   to skip that check.  err receives the reference's message. */
int oracle_append_pages(size_t elem_size, void* key_pool, void* value_pool, int64_t page_count, int num_kv_heads,
                        int page_size, int head_dim, const int64_t* page_ids, int64_t num_page_ids,
                        int cached_token_count, const void* key, const void* value, int token_count,
                        const uint8_t* page_writable, char* err, size_t errlen);

/* A packed batch in the library's layout (all strides in elements):
   q [Hq, total_q, D], k and v [Hkv, total_q, D] as produced by the Q/K/V
   projections (common.rs:268-283); int32 block tables [num_seqs,
   max_pages_per_seq] already holding the pages this append writes;
   seq_lens = cached_token_count after the append; cu_q_lens = prefix sums of
   q_len.  Request b's new tokens sit at positions seq_lens[b] - q_len ..
   seq_lens[b] - 1.  Writes the rotated queries to q_out and the rotated keys
   and the values into the pools. */
typedef struct {
  int dtype, rope_type;
  int num_seqs, num_q_heads, num_kv_heads, head_dim, page_size;
  int64_t num_pages;
  int max_pages_per_seq;
  const void* q;
  int64_t q_stride_head, q_stride_token;
  const void* k;
  int64_t k_stride_head, k_stride_token;
  const void* v;
  int64_t v_stride_head, v_stride_token;
  const void* cos_table;
  const void* sin_table;
  int rope_len;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  const int32_t* cu_q_lens;
  void* q_out;
  int64_t q_out_stride_head, q_out_stride_token;
  void* key_pool;
  void* value_pool;
} oracle_rope_append_batch;

/* forward_attention's per-request loop up to the attention call
   (common.rs:285-320): narrow, RoPE on Q and K, append K/V. */
int oracle_rope_append(const oracle_rope_append_batch* b, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif
