/*
 * ORACLE — test infrastructure only (see paged_attention_oracle.c).
 * CPU restatement of mini-vllm-rs page-wise attention
 * (src/models/backends/common.rs:739-978); never linked into the product.
 */
#ifndef MVR_PAGED_ATTENTION_ORACLE_H
#define MVR_PAGED_ATTENTION_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F32 = 0, ORACLE_F16 = 1 };

/* Modes: the reference dataflow with concatenated V (common.rs:805-816, the
   default), the page-wise V variant (common.rs:797-804), or an independent
   double-precision evaluation of the same attention. */
enum { ORACLE_REF_CONCAT_V = 0, ORACLE_REF_PAGEWISE_V = 1, ORACLE_EXACT_F64 = 2 };

enum {
  ORACLE_OK = 0,
  ORACLE_E_INVALID = -1,
  ORACLE_E_LENGTH = -2,    /* cached_token_count != cached_kv_len + q_len */
  ORACLE_E_UNCOVERED = -3, /* pages do not cover the sequence length */
  ORACLE_E_PAGE_ID = -4,   /* page id outside the pool */
  ORACLE_E_NO_PAGES = -5,
  ORACLE_E_ALLOC = -6
};

/* AttentionDimensions (common.rs:189-206) plus the activation dtype. */
typedef struct {
  int dtype;
  int num_q_heads;
  int num_kv_heads;
  int head_dim;
  int cached_kv_len;
  int q_len;
} oracle_dims;

uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);

/* forward_paged_attention for one request.  request_q: [1, Hq, q_len, D]
   contiguous in dtype; pools [page_count, 1, Hkv, P, D]; request_y receives
   [Hq, q_len, D] as double.  Error text mirrors the reference's messages. */
int oracle_forward_paged_attention(const oracle_dims* dims, const void* request_q, const void* key_pool,
                                   const void* value_pool, int64_t page_count, const int64_t* page_ids,
                                   int64_t num_page_ids, int per_page_token_count, int cached_token_count, int mode,
                                   double* request_y, char* err, size_t errlen);

/* forward_contiguous_attention: K/V [1, Hkv, kv_len, D]. */
int oracle_forward_contiguous_attention(const oracle_dims* dims, const void* request_q, const void* full_k,
                                        const void* full_v, int kv_len, int mode, double* request_y);

/* reconstruct_contiguous_tensor: gathers [Hkv, L, D] from a pool. */
int oracle_reconstruct_contiguous(int dtype, const void* pool, int num_kv_heads, int page_size, int head_dim,
                                  int64_t page_count, const int64_t* page_ids, int64_t num_page_ids,
                                  int cached_token_count, void* out);

/* A packed batch in the library's layout: q/out [Hq, total_q, D] through
   strides (elements), int32 block tables [num_seqs, max_pages_per_seq],
   seq_lens = cached_token_count per sequence (current query included),
   cu_q_lens = prefix sums of q_len. */
typedef struct {
  int dtype;
  int num_seqs, num_q_heads, num_kv_heads, head_dim, page_size;
  int64_t num_pages;
  int max_pages_per_seq;
  const void* q;
  int64_t q_stride_head, q_stride_token;
  const void* key_pool;
  const void* value_pool;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  const int32_t* cu_q_lens;
} oracle_batch;

/* out: [Hq][total_q][D] double.  OpenMP over (sequence, kv head). */
int oracle_paged_attention(const oracle_batch* b, int mode, int num_threads, double* out);

int oracle_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
