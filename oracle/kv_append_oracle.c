/*
 * ORACLE — test infrastructure only.
 *
 * CPU restatement of the two steps mini-vllm-rs runs for each request just
 * before its attention call, used as the parity checker for the library's
 * fused RoPE + KV-append kernel.  Only the test suite may load it.
 *
 * What is restated (reference paths relative to the mini-vllm-rs tree):
 *   - per-request narrow of packed Q/K/V      src/models/backends/common.rs:294-305
 *   - forward_rope                            src/models/backends/common.rs:344-359
 *   - RotaryEmbeddingType                     src/models/backends/common.rs:552-556
 *   - append_new_key_value                    src/model_runner/server/kv_cache/paged_cache.rs:170-199
 *   - validate_cache_append                   src/model_runner/server/kv_cache/utils.rs:13-38
 *   - append_to_pages                         src/model_runner/server/kv_cache/paged_cache.rs:290-327
 *   - PhysicalPagePool::write_page            src/model_runner/server/kv_cache/physical_page_pool.rs:188-209
 *   - PageState::is_writable                  src/model_runner/server/kv_cache/physical_page_pool.rs:57-59
 *
 * The rotation itself is candle-nn 0.11.1's CPU rope / rope_i (a crate
 * dependency, absent here), restated from its published algorithm: for a
 * row x of head_dim D at position p and i < D/2, with c = cos[p][i],
 * s = sin[p][i],
 *   Neox:        y[i] = x[i]*c - x[i+D/2]*s,  y[i+D/2] = x[i]*s + x[i+D/2]*c
 *   Interleaved: y[2i] = x[2i]*c - x[2i+1]*s, y[2i+1] = x[2i]*s + x[2i+1]*c
 * evaluated in the activation dtype T, each product and the sum rounded to T
 * (half 2.7.1 widens f16 operands to f32 and rounds every result back to f16
 * with round-to-nearest-even; f32 products are not fused).
 */
#include "kv_append_oracle.h"

#include "paged_attention_oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float ld(const void* base, size_t i, int dtype) {
  return dtype == ORACLE_F16 ? oracle_f16_to_f32(((const uint16_t*)base)[i]) : ((const float*)base)[i];
}

static void st(void* base, size_t i, int dtype, float v) {
  if (dtype == ORACLE_F16)
    ((uint16_t*)base)[i] = oracle_f32_to_f16(v);
  else
    ((float*)base)[i] = v;
}

/* One arithmetic result stored in T. */
static float rt(float v, int dtype) { return dtype == ORACLE_F16 ? oracle_f16_to_f32(oracle_f32_to_f16(v)) : v; }

/* Element indices of rotation pair i of a row (common.rs:355-358 selects the
   candle kernel by RotaryEmbeddingType). */
static void pair_index(int rope_type, int head_dim, int i, int* a, int* b) {
  if (rope_type == ORACLE_ROPE_NEOX) {
    *a = i;
    *b = i + head_dim / 2;
  } else {
    *a = 2 * i;
    *b = 2 * i + 1;
  }
}

int oracle_rope(int dtype, int rope_type, const void* x, int heads, int q_len, int head_dim, const void* cos_table,
                const void* sin_table, int rope_len, int start_pos, void* y) {
  if (head_dim <= 0 || head_dim % 2 || heads < 0 || q_len < 0 || start_pos < 0) return ORACLE_APPEND_E_INVALID;
  if (rope_type != ORACLE_ROPE_NEOX && rope_type != ORACLE_ROPE_INTERLEAVED) return ORACLE_APPEND_E_INVALID;
  if (start_pos + q_len > rope_len) return ORACLE_APPEND_E_ROPE_RANGE;
  const int half = head_dim / 2;
  for (int h = 0; h < heads; h++)
    for (int t = 0; t < q_len; t++) {
      const size_t row = ((size_t)h * q_len + t) * head_dim;
      const size_t cs = (size_t)(start_pos + t) * half;
      for (int i = 0; i < half; i++) {
        int a, b;
        pair_index(rope_type, head_dim, i, &a, &b);
        const float xa = ld(x, row + a, dtype), xb = ld(x, row + b, dtype);
        const float c = ld(cos_table, cs + i, dtype), s = ld(sin_table, cs + i, dtype);
        const float ya = rt(rt(xa * c, dtype) - rt(xb * s, dtype), dtype);
        const float yb = rt(rt(xa * s, dtype) + rt(xb * c, dtype), dtype);
        st(y, row + a, dtype, ya);
        st(y, row + b, dtype, yb);
      }
    }
  return ORACLE_APPEND_OK;
}

int oracle_rope_f64(int rope_type, const double* x, int heads, int q_len, int head_dim, const double* cos_table,
                    const double* sin_table, int rope_len, int start_pos, double* y) {
  if (head_dim <= 0 || head_dim % 2 || heads < 0 || q_len < 0 || start_pos < 0) return ORACLE_APPEND_E_INVALID;
  if (rope_type != ORACLE_ROPE_NEOX && rope_type != ORACLE_ROPE_INTERLEAVED) return ORACLE_APPEND_E_INVALID;
  if (start_pos + q_len > rope_len) return ORACLE_APPEND_E_ROPE_RANGE;
  const int half = head_dim / 2;
  for (int h = 0; h < heads; h++)
    for (int t = 0; t < q_len; t++) {
      const size_t row = ((size_t)h * q_len + t) * head_dim;
      const size_t cs = (size_t)(start_pos + t) * half;
      for (int i = 0; i < half; i++) {
        int a, b;
        pair_index(rope_type, head_dim, i, &a, &b);
        const double xa = x[row + a], xb = x[row + b], c = cos_table[cs + i], s = sin_table[cs + i];
        y[row + a] = xa * c - xb * s;
        y[row + b] = xa * s + xb * c;
      }
    }
  return ORACLE_APPEND_OK;
}

int oracle_append_pages(size_t elem_size, void* key_pool, void* value_pool, int64_t page_count, int num_kv_heads,
                        int page_size, int head_dim, const int64_t* page_ids, int64_t num_page_ids,
                        int cached_token_count, const void* key, const void* value, int token_count,
                        const uint8_t* page_writable, char* err, size_t errlen) {
  if (err && errlen) err[0] = 0;
  if (elem_size == 0 || page_size <= 0 || head_dim <= 0 || num_kv_heads <= 0 || cached_token_count < 0)
    return ORACLE_APPEND_E_INVALID;
  if (token_count <= 0) {
    if (err && errlen) snprintf(err, errlen, "cannot append an empty KV-cache tensor");
    return ORACLE_APPEND_E_EMPTY;
  }
  const size_t row_bytes = (size_t)head_dim * elem_size;
  int cached = cached_token_count;
  int input_offset = 0;
  /* append_to_pages: fill the partial last page, then one page at a time. */
  while (input_offset < token_count) {
    const int page_offset = cached % page_size;
    const int64_t page_index = cached / page_size;
    if (page_index >= num_page_ids) {
      if (err && errlen) snprintf(err, errlen, "partial KV-cache page is missing from the block table");
      return ORACLE_APPEND_E_MISSING;
    }
    const int64_t page = page_ids[page_index];
    if (page < 0 || page >= page_count) {
      if (err && errlen) snprintf(err, errlen, "page id %lld is outside the pool of %lld pages", (long long)page,
                                  (long long)page_count);
      return ORACLE_APPEND_E_PAGE_ID;
    }
    int written = page_size - page_offset;
    if (written > token_count - input_offset) written = token_count - input_offset;
    /* write_page: only PendingWrite pages may be mutated. */
    if (page_writable && !page_writable[page]) {
      if (err && errlen) snprintf(err, errlen, "cannot mutate written physical page %lld", (long long)page);
      return ORACLE_APPEND_E_READ_ONLY;
    }
    /* key.narrow(2, input_offset, written) -> page[:, :, page_offset.., :] */
    for (int h = 0; h < num_kv_heads; h++)
      for (int t = 0; t < written; t++) {
        const size_t src = ((size_t)h * token_count + input_offset + t) * row_bytes;
        const size_t dst = (((size_t)page * num_kv_heads + h) * page_size + page_offset + t) * row_bytes;
        memcpy((char*)key_pool + dst, (const char*)key + src, row_bytes);
        memcpy((char*)value_pool + dst, (const char*)value + src, row_bytes);
      }
    cached += written;
    input_offset += written;
  }
  return ORACLE_APPEND_OK;
}

/* Copies rows [heads][q_len][D] between a strided packed tensor and a
   contiguous request tensor (the narrow(...).contiguous() of common.rs:299-305). */
static void gather_rows(const void* src, int64_t stride_head, int64_t stride_token, int heads, int q_start, int q_len,
                        int head_dim, size_t es, void* dst) {
  for (int h = 0; h < heads; h++)
    for (int t = 0; t < q_len; t++)
      memcpy((char*)dst + ((size_t)h * q_len + t) * head_dim * es,
             (const char*)src + ((size_t)h * stride_head + (size_t)(q_start + t) * stride_token) * es, head_dim * es);
}

static void scatter_rows(const void* src, int heads, int q_start, int q_len, int head_dim, size_t es, void* dst,
                         int64_t stride_head, int64_t stride_token) {
  for (int h = 0; h < heads; h++)
    for (int t = 0; t < q_len; t++)
      memcpy((char*)dst + ((size_t)h * stride_head + (size_t)(q_start + t) * stride_token) * es,
             (const char*)src + ((size_t)h * q_len + t) * head_dim * es, head_dim * es);
}

int oracle_rope_append(const oracle_rope_append_batch* b, char* err, size_t errlen) {
  if (err && errlen) err[0] = 0;
  if (!b || b->num_seqs <= 0 || b->head_dim <= 0 || b->num_kv_heads <= 0 || b->num_q_heads % b->num_kv_heads)
    return ORACLE_APPEND_E_INVALID;
  const size_t es = b->dtype == ORACLE_F16 ? 2 : 4;
  const int D = b->head_dim;
  int rc = ORACLE_APPEND_OK;
  int max_q = 0;
  for (int s = 0; s < b->num_seqs; s++) {
    const int ql = b->cu_q_lens[s + 1] - b->cu_q_lens[s];
    if (ql > max_q) max_q = ql;
  }
  const size_t qbytes = (size_t)b->num_q_heads * (max_q > 0 ? max_q : 1) * D * es;
  const size_t kbytes = (size_t)b->num_kv_heads * (max_q > 0 ? max_q : 1) * D * es;
  char* rq = malloc(qbytes);
  char* rk = malloc(kbytes);
  char* rv = malloc(kbytes);
  int64_t* ids = malloc(sizeof(int64_t) * (size_t)(b->max_pages_per_seq > 0 ? b->max_pages_per_seq : 1));
  if (!rq || !rk || !rv || !ids) {
    rc = ORACLE_APPEND_E_INVALID;
    goto done;
  }
  for (int s = 0; s < b->num_seqs && rc == ORACLE_APPEND_OK; s++) {
    const int q_start = b->cu_q_lens[s];
    const int q_len = b->cu_q_lens[s + 1] - q_start;
    const int start_pos = b->seq_lens[s] - q_len; /* == cached_kv_len == start_pos (utils.rs:20-24) */
    if (q_len <= 0) {
      if (err && errlen) snprintf(err, errlen, "cannot append an empty KV-cache tensor");
      rc = ORACLE_APPEND_E_EMPTY;
      break;
    }
    if (start_pos < 0) {
      rc = ORACLE_APPEND_E_INVALID;
      break;
    }
    gather_rows(b->q, b->q_stride_head, b->q_stride_token, b->num_q_heads, q_start, q_len, D, es, rq);
    gather_rows(b->k, b->k_stride_head, b->k_stride_token, b->num_kv_heads, q_start, q_len, D, es, rk);
    gather_rows(b->v, b->v_stride_head, b->v_stride_token, b->num_kv_heads, q_start, q_len, D, es, rv);
    rc = oracle_rope(b->dtype, b->rope_type, rq, b->num_q_heads, q_len, D, b->cos_table, b->sin_table, b->rope_len,
                     start_pos, rq);
    if (rc == ORACLE_APPEND_OK)
      rc = oracle_rope(b->dtype, b->rope_type, rk, b->num_kv_heads, q_len, D, b->cos_table, b->sin_table,
                       b->rope_len, start_pos, rk);
    if (rc != ORACLE_APPEND_OK) {
      if (rc == ORACLE_APPEND_E_ROPE_RANGE && err && errlen)
        snprintf(err, errlen, "rotary tables hold %d positions, request needs %d", b->rope_len, start_pos + q_len);
      break;
    }
    scatter_rows(rq, b->num_q_heads, q_start, q_len, D, es, b->q_out, b->q_out_stride_head, b->q_out_stride_token);
    const int n_ids = (b->seq_lens[s] + b->page_size - 1) / b->page_size;
    if (n_ids > b->max_pages_per_seq) {
      if (err && errlen) snprintf(err, errlen, "partial KV-cache page is missing from the block table");
      rc = ORACLE_APPEND_E_MISSING;
      break;
    }
    for (int i = 0; i < n_ids; i++) ids[i] = b->block_tables[(size_t)s * b->max_pages_per_seq + i];
    rc = oracle_append_pages(es, b->key_pool, b->value_pool, b->num_pages, b->num_kv_heads, b->page_size, D, ids,
                             n_ids, start_pos, rk, rv, q_len, NULL, err, errlen);
  }
done:
  free(rq);
  free(rk);
  free(rv);
  free(ids);
  return rc;
}
