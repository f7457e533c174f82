/*
 * ORACLE — test infrastructure only.
 *
 * CPU restatement of mini-vllm-rs's page-wise attention, used as the parity
 * checker for the HIP library and as the timed CPU baseline.  Only the test
 * suite, the smoke check and the benchmark's CPU-baseline leg may load this
 * library; the product library (libmvr_attn.so) never calls it.
 *
 * What is restated (reference paths relative to the mini-vllm-rs tree):
 *   - forward_paged_attention          src/models/backends/common.rs:739-817
 *   - get_page_slice_from_pool         src/models/backends/common.rs:967-978
 *   - matmul_query_key (grouped)       src/models/backends/common.rs:828-859
 *   - scale by 1/sqrt(head_dim)        src/models/backends/common.rs:784-785
 *   - apply_causal_attention_mask      src/models/backends/common.rs:948-965
 *   - softmax_last_dim                 called at common.rs:794 (candle-nn 0.11.1)
 *   - matmul_attention_value           src/models/backends/common.rs:870-906
 *   - matmul_paged_attention_value     src/models/backends/common.rs:914-946
 *   - forward_contiguous_attention     src/models/backends/common.rs:703-737
 *   - reconstruct_contiguous_tensor    src/model_runner/server/kv_cache/paged_cache.rs:363-391
 *   - length checks                    common.rs:447-454, common.rs:776-781
 *
 * Pool layout (src/models/mod.rs:56-65, kv_cache/utils.rs:55-74):
 *   [page_count, 1, num_kv_heads, per_page_token_count, head_dim]; element
 *   (page p, kv head h, slot t, dim d) is at ((p*Hkv + h)*P + t)*D + d.
 *
 * Dtype semantics.  The reference runs each step as a Candle op whose result
 * is stored in the activation dtype (F32 or F16).  Candle 0.11.1 is a crate
 * dependency that is absent here, so its published CPU algorithms are
 * restated, not read:
 *   - matmul (gemm 0.19): products summed in f32, result rounded to T;
 *   - Tensor / f64 = affine(1/x, 0): mul = T(1/x), v*mul + 0 in T;
 *   - where_cond(mask, -inf, scores): select;
 *   - softmax_last_dim: max in T, e = T(exp(T(s - max))), sum of e in f32
 *     rounded to T, e / sum in T;
 *   - f16 arithmetic (half 2.x): operands widened to f32, result rounded to
 *     f16 with round-to-nearest-even.
 * The reduction order inside Candle's gemm / reductions is not pinned; sums
 * here run in index order.  Mode ORACLE_EXACT_F64 drops every rounding and
 * evaluates the same attention in double precision, as an independent check.
 */
#include "paged_attention_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- f16 ---- */

uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf / nan */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  if (ax >= 0x38800000u) {                                  /* normal f16 */
    uint32_t r = ax - 0x38000000u;                           /* rebias 127 -> 15 */
    r += 0xfffu + ((r >> 13) & 1u);                          /* RNE on 13 dropped bits */
    return (uint16_t)(sign | (r >> 13));
  }
  /* subnormal f16 (or zero): value = q * 2^-24, q = round(mant24 * 2^(e-126)) */
  uint32_t e = ax >> 23;
  if (e < 102u) return (uint16_t)sign; /* below 2^-25: rounds to zero */
  uint32_t m = (ax & 0x7fffffu) | 0x800000u;
  uint32_t shift = 126u - e; /* 14 .. 24 */
  uint32_t q = m >> shift;
  uint32_t rem = m & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else { /* subnormal: normalise */
      int k = -1;
      do {
        m <<= 1;
        k++;
      } while (!(m & 0x400u));
      x = sign | ((uint32_t)(112 - k) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

/* Rounds a float to the storage dtype and back (identity for F32). */
static inline float round_t(float v, int dtype) {
  return dtype == ORACLE_F16 ? oracle_f16_to_f32(oracle_f32_to_f16(v)) : v;
}

static inline float load_t(const void* base, size_t idx, int dtype) {
  if (dtype == ORACLE_F16) return oracle_f16_to_f32(((const uint16_t*)base)[idx]);
  return ((const float*)base)[idx];
}

/* ------------------------------------------------------------- errors ---- */

static void set_err(char* err, size_t errlen, const char* fmt, long a, long b) {
  if (err && errlen) snprintf(err, errlen, fmt, a, b);
}

/* ------------------------------------------------ one (request, kv head) ---- */

/*
 * Attention for one request and one KV head group, following
 * forward_paged_attention (common.rs:739-817) with grouped Q rows
 * (common.rs:846-858: Q [Hkv, rep*q, D] x K^T; rows of one KV head are the
 * consecutive Q heads h*rep .. h*rep+rep-1).
 *
 * q_at(r, i, d) reads Q head (kv_head*rep + r), query position i.
 * Output y[(r*q_len + i)*D + d] as double (exactly the T-rounded value in the
 * reference dataflow modes).
 */
typedef struct {
  int dtype;
  int Hq, Hkv, D, P;
  int cached_kv_len, q_len;
  const void* q;
  int64_t q_stride_head, q_stride_token; /* elements */
  const void* kpool;
  const void* vpool;
  const int64_t* page_ids; /* logical -> physical */
  int64_t num_page_ids;
  int64_t page_count;
  int cached_token_count;
} group_ctx;

static size_t pool_index(const group_ctx* c, int64_t page, int h, int t, int d) {
  return (((size_t)page * c->Hkv + h) * c->P + t) * c->D + d;
}

/* The reference's checks on the page list (common.rs:758-781): every page
   that holds keys lies inside the pool, and the pages cover the length. */
static int check_page_list(const group_ctx* c) {
  int remaining = c->cached_token_count;
  for (int64_t pi = 0; pi < c->num_page_ids; pi++) {
    const int slice = remaining < c->P ? remaining : c->P;
    const int64_t page = c->page_ids[pi];
    if (slice > 0 && (page < 0 || page >= c->page_count)) return ORACLE_E_PAGE_ID;
    remaining -= slice;
  }
  return remaining == 0 ? 0 : ORACLE_E_UNCOVERED;
}

/* Returns 0 or ORACLE_E_*; writes one group's output rows. */
static int attend_group(const group_ctx* c, int kv_head, int mode, double* y /* [rep*q][D] */,
                        float* scratch /* [rep*q][L] */, float* vcat /* [L][D] */) {
  const int rep = c->Hq / c->Hkv;
  const int q_len = c->q_len, D = c->D, L = c->cached_token_count;
  const int rows = rep * q_len;
  const int dtype = c->dtype;

  if (mode == ORACLE_EXACT_F64) {
    /* Independent double-precision attention: no per-op rounding.  It reads
       the pool through the same page list, so the same checks come first. */
    const int pc = check_page_list(c);
    if (pc != 0) return pc;
    double* s = (double*)malloc(sizeof(double) * (size_t)(L > 0 ? L : 1));
    if (!s) return ORACLE_E_ALLOC;
    const double scale = 1.0 / sqrt((double)D);
    for (int r = 0; r < rep; r++) {
      for (int i = 0; i < q_len; i++) {
        const int qh = kv_head * rep + r;
        const int limit = c->cached_kv_len + i; /* key j visible iff j <= c + i */
        double mx = -INFINITY;
        for (int j = 0; j < L; j++) {
          const int64_t page = c->page_ids[j / c->P];
          const int slot = j % c->P;
          double acc = 0.0;
          for (int d = 0; d < D; d++) {
            acc += (double)load_t(c->q, (size_t)qh * c->q_stride_head + (size_t)i * c->q_stride_token + d, dtype) *
                   (double)load_t(c->kpool, pool_index(c, page, kv_head, slot, d), dtype);
          }
          s[j] = j <= limit ? acc * scale : -INFINITY;
          if (s[j] > mx) mx = s[j];
        }
        double sum = 0.0;
        for (int j = 0; j < L; j++) {
          s[j] = j <= limit ? exp(s[j] - mx) : 0.0;
          sum += s[j];
        }
        double* out = y + (size_t)(r * q_len + i) * D;
        for (int d = 0; d < D; d++) out[d] = 0.0;
        for (int j = 0; j < L; j++) {
          if (s[j] == 0.0) continue;
          const int64_t page = c->page_ids[j / c->P];
          const int slot = j % c->P;
          const double w = s[j] / sum;
          for (int d = 0; d < D; d++) out[d] += w * (double)load_t(c->vpool, pool_index(c, page, kv_head, slot, d), dtype);
        }
      }
    }
    free(s);
    return 0;
  }

  /* --- reference dataflow (common.rs:758-775): per-page score slices --- */
  /* Q rows of this kv head, widened once: row r*q_len + i is Q head
     kv_head*rep + r at position i (grouped layout, common.rs:846-858). */
  float* qf = (float*)malloc(sizeof(float) * (size_t)rows * D);
  float* kf = (float*)malloc(sizeof(float) * (size_t)D);
  if (!qf || !kf) {
    free(qf);
    free(kf);
    return ORACLE_E_ALLOC;
  }
  for (int r = 0; r < rep; r++)
    for (int i = 0; i < q_len; i++)
      for (int d = 0; d < D; d++)
        qf[(size_t)(r * q_len + i) * D + d] =
            load_t(c->q, (size_t)(kv_head * rep + r) * c->q_stride_head + (size_t)i * c->q_stride_token + d, dtype);
  int remaining = L;
  int col = 0;
  for (int64_t pi = 0; pi < c->num_page_ids; pi++) {
    const int slice = remaining < c->P ? remaining : c->P; /* common.rs:759 */
    const int64_t page = c->page_ids[pi];
    /* narrow(0, page_id, 1) on the pool fails for an out-of-range page. */
    if (slice > 0 && (page < 0 || page >= c->page_count)) {
      free(qf);
      free(kf);
      return ORACLE_E_PAGE_ID;
    }
    for (int t = 0; t < slice; t++) {
      for (int d = 0; d < D; d++) kf[d] = load_t(c->kpool, pool_index(c, page, kv_head, t, d), dtype);
      for (int row = 0; row < rows; row++) {
        const float* qr = qf + (size_t)row * D;
        float acc = 0.0f; /* gemm: f32 sum of products, rounded to T */
        for (int d = 0; d < D; d++) acc += qr[d] * kf[d];
        scratch[(size_t)row * L + col + t] = round_t(acc, dtype);
      }
      /* V slice for the concatenated path (common.rs:808). */
      for (int d = 0; d < D; d++) vcat[(size_t)(col + t) * D + d] = load_t(c->vpool, pool_index(c, page, kv_head, t, d), dtype);
    }
    col += slice;
    remaining -= slice;
  }
  free(qf);
  free(kf);
  if (remaining != 0) return ORACLE_E_UNCOVERED; /* common.rs:776-781 */

  /* Scale: Tensor / f64 -> affine(1/sqrt(D), 0) in T (common.rs:784-785). */
  const float mul = round_t((float)(1.0 / sqrt((double)D)), dtype);
  for (int row = 0; row < rows; row++) {
    const int i = row % q_len;
    const int limit = c->cached_kv_len + i;
    float* s = scratch + (size_t)row * L;
    for (int j = 0; j < L; j++) {
      float v = round_t(round_t(s[j] * mul, dtype) + 0.0f, dtype);
      s[j] = j <= limit ? v : -INFINITY; /* common.rs:948-965 */
    }
    /* softmax_last_dim */
    float mx = -INFINITY;
    for (int j = 0; j < L; j++) mx = s[j] > mx ? s[j] : mx;
    float sum = 0.0f;
    for (int j = 0; j < L; j++) {
      s[j] = round_t(expf(round_t(s[j] - mx, dtype)), dtype);
      sum += s[j];
    }
    sum = round_t(sum, dtype);
    for (int j = 0; j < L; j++) s[j] = round_t(s[j] / sum, dtype);
  }

  if (mode == ORACLE_REF_PAGEWISE_V) {
    /* matmul_paged_attention_value (common.rs:914-946): one product per page,
       partial outputs summed in T. */
    float* part = (float*)malloc(sizeof(float) * (size_t)rows * D);
    float* accum = (float*)malloc(sizeof(float) * (size_t)rows * D);
    if (!part || !accum) {
      free(part);
      free(accum);
      return ORACLE_E_ALLOC;
    }
    int start = 0, first = 1;
    remaining = L;
    for (int64_t pi = 0; pi < c->num_page_ids; pi++) {
      const int slice = remaining < c->P ? remaining : c->P;
      for (int row = 0; row < rows; row++) {
        for (int d = 0; d < D; d++) {
          float acc = 0.0f;
          for (int t = 0; t < slice; t++) acc += scratch[(size_t)row * L + start + t] * vcat[(size_t)(start + t) * D + d];
          part[(size_t)row * D + d] = round_t(acc, dtype);
        }
      }
      for (size_t k = 0; k < (size_t)rows * D; k++) accum[k] = first ? part[k] : round_t(accum[k] + part[k], dtype);
      first = 0;
      start += slice;
      remaining -= slice;
    }
    if (first) {
      free(part);
      free(accum);
      return ORACLE_E_NO_PAGES; /* common.rs:943-945 */
    }
    for (size_t k = 0; k < (size_t)rows * D; k++) y[k] = accum[k];
    free(part);
    free(accum);
    return 0;
  }

  /* Concatenated V (common.rs:805-816, the default).  Each output element
     sums its products in key order j = 0 .. L-1 in f32, then rounds to T. */
  float* acc = (float*)malloc(sizeof(float) * (size_t)D);
  if (!acc) return ORACLE_E_ALLOC;
  for (int row = 0; row < rows; row++) {
    for (int d = 0; d < D; d++) acc[d] = 0.0f;
    const float* w = scratch + (size_t)row * L;
    for (int j = 0; j < L; j++) {
      const float wj = w[j];
      const float* vj = vcat + (size_t)j * D;
      for (int d = 0; d < D; d++) acc[d] += wj * vj[d];
    }
    for (int d = 0; d < D; d++) y[(size_t)row * D + d] = round_t(acc[d], dtype);
  }
  free(acc);
  return 0;
}

/* -------------------------------------------------- request-level API ---- */

int oracle_forward_paged_attention(const oracle_dims* dims, const void* request_q, const void* key_pool,
                                   const void* value_pool, int64_t page_count, const int64_t* page_ids,
                                   int64_t num_page_ids, int per_page_token_count, int cached_token_count, int mode,
                                   double* request_y, char* err, size_t errlen) {
  if (!dims || dims->num_kv_heads <= 0 || dims->num_q_heads % dims->num_kv_heads != 0 || dims->head_dim <= 0 ||
      dims->q_len <= 0 || per_page_token_count <= 0) {
    set_err(err, errlen, "invalid attention dimensions (%ld, %ld)", dims ? dims->num_q_heads : -1,
            dims ? dims->num_kv_heads : -1);
    return ORACLE_E_INVALID;
  }
  const long expected = (long)dims->cached_kv_len + dims->q_len;
  if (cached_token_count != expected) { /* common.rs:447-454 */
    set_err(err, errlen, "paged KV cache reports sequence length %ld, expected %ld", (long)cached_token_count,
            expected);
    return ORACLE_E_LENGTH;
  }
  group_ctx c;
  c.dtype = dims->dtype;
  c.Hq = dims->num_q_heads;
  c.Hkv = dims->num_kv_heads;
  c.D = dims->head_dim;
  c.P = per_page_token_count;
  c.cached_kv_len = dims->cached_kv_len;
  c.q_len = dims->q_len;
  c.q = request_q;
  c.q_stride_head = (int64_t)dims->q_len * dims->head_dim; /* [1, Hq, q, D] contiguous */
  c.q_stride_token = dims->head_dim;
  c.kpool = key_pool;
  c.vpool = value_pool;
  c.page_ids = page_ids;
  c.num_page_ids = num_page_ids;
  c.page_count = page_count;
  c.cached_token_count = cached_token_count;

  const int rep = c.Hq / c.Hkv;
  const int rows = rep * c.q_len;
  const int L = cached_token_count;
  float* scratch = (float*)malloc(sizeof(float) * (size_t)rows * (L > 0 ? L : 1));
  float* vcat = (float*)malloc(sizeof(float) * (size_t)(L > 0 ? L : 1) * c.D);
  double* y = (double*)malloc(sizeof(double) * (size_t)rows * c.D);
  if (!scratch || !vcat || !y) {
    free(scratch);
    free(vcat);
    free(y);
    return ORACLE_E_ALLOC;
  }
  int rc = 0;
  for (int h = 0; h < c.Hkv && rc == 0; h++) {
    rc = attend_group(&c, h, mode, y, scratch, vcat);
    if (rc == 0) {
      for (int r = 0; r < rep; r++)
        for (int i = 0; i < c.q_len; i++)
          for (int d = 0; d < c.D; d++)
            request_y[((size_t)(h * rep + r) * c.q_len + i) * c.D + d] = y[(size_t)(r * c.q_len + i) * c.D + d];
    }
  }
  if (rc == ORACLE_E_UNCOVERED) {
    long covered = 0, rem = L;
    for (int64_t pi = 0; pi < num_page_ids; pi++) {
      long s = rem < per_page_token_count ? rem : per_page_token_count;
      covered += s;
      rem -= s;
    }
    set_err(err, errlen, "paged KV cache contains fewer pages than its sequence length, leaving %ld tokens uncovered",
            (long)L - covered, 0);
  } else if (rc == ORACLE_E_PAGE_ID) {
    set_err(err, errlen, "page id out of range for a pool of %ld pages%.0ld", (long)page_count, 0);
  } else if (rc == ORACLE_E_NO_PAGES) {
    set_err(err, errlen, "paged KV cache contains no value pages%.0ld%.0ld", 0, 0);
  }
  free(scratch);
  free(vcat);
  free(y);
  return rc;
}

/* ---------------------------------------------------- contiguous path ---- */

int oracle_forward_contiguous_attention(const oracle_dims* dims, const void* request_q, const void* full_k,
                                        const void* full_v, int kv_len, int mode, double* request_y) {
  /* forward_contiguous_attention (common.rs:703-737) over K/V [1,Hkv,L,D]:
     identical to the paged path over one page of L tokens, so it reuses it. */
  if (kv_len != dims->cached_kv_len + dims->q_len) return ORACLE_E_LENGTH; /* common.rs:391-398 */
  int64_t page = 0;
  return oracle_forward_paged_attention(dims, request_q, full_k, full_v, 1, &page, 1, kv_len > 0 ? kv_len : 1, kv_len,
                                        mode, request_y, NULL, 0);
}

/* ---------------------------------------------- reconstruct (gather) ---- */

int oracle_reconstruct_contiguous(int dtype, const void* pool, int num_kv_heads, int page_size, int head_dim,
                                  int64_t page_count, const int64_t* page_ids, int64_t num_page_ids,
                                  int cached_token_count, void* out /* [Hkv, L, D] */) {
  /* paged_cache.rs:363-391: narrow every page to its valid tokens, cat on the
     token axis.  Pure data movement, so the copy is bit-exact. */
  if (cached_token_count <= 0 || num_page_ids <= 0) return ORACLE_E_NO_PAGES;
  const size_t es = dtype == ORACLE_F16 ? 2 : 4;
  int remaining = cached_token_count, col = 0;
  for (int64_t pi = 0; pi < num_page_ids; pi++) {
    const int slice = remaining < page_size ? remaining : page_size;
    const int64_t page = page_ids[pi];
    if (slice > 0 && (page < 0 || page >= page_count)) return ORACLE_E_PAGE_ID;
    for (int h = 0; h < num_kv_heads; h++)
      for (int t = 0; t < slice; t++) {
        const size_t src = (((size_t)page * num_kv_heads + h) * page_size + t) * head_dim;
        const size_t dst = ((size_t)h * cached_token_count + col + t) * head_dim;
        memcpy((char*)out + dst * es, (const char*)pool + src * es, es * head_dim);
      }
    col += slice;
    remaining -= slice;
  }
  return remaining == 0 ? 0 : ORACLE_E_UNCOVERED;
}

/* ------------------------------------------------------ batched API ---- */

int oracle_paged_attention(const oracle_batch* b, int mode, int num_threads, double* out /* [Hq][total_q][D] */) {
  if (!b || b->num_seqs <= 0 || b->num_kv_heads <= 0 || b->num_q_heads % b->num_kv_heads != 0) return ORACLE_E_INVALID;
  const int rep = b->num_q_heads / b->num_kv_heads;
  const int total_q = b->cu_q_lens[b->num_seqs];
  const int n_items = b->num_seqs * b->num_kv_heads;
  int rc_all = 0;
#ifdef _OPENMP
  if (num_threads > 0) omp_set_num_threads(num_threads);
#pragma omp parallel for schedule(dynamic, 1) reduction(| : rc_all)
#endif
  for (int item = 0; item < n_items; item++) {
    const int s = item / b->num_kv_heads, h = item % b->num_kv_heads;
    const int q0 = b->cu_q_lens[s], q_len = b->cu_q_lens[s + 1] - q0;
    const int L = b->seq_lens[s];
    if (q_len <= 0 || L < q_len) {
      rc_all |= 1;
      continue;
    }
    const int npages = b->max_pages_per_seq;
    int64_t* ids = (int64_t*)malloc(sizeof(int64_t) * (size_t)npages);
    const int need = (L + b->page_size - 1) / b->page_size;
    group_ctx c;
    c.dtype = b->dtype;
    c.Hq = b->num_q_heads;
    c.Hkv = b->num_kv_heads;
    c.D = b->head_dim;
    c.P = b->page_size;
    c.cached_kv_len = L - q_len;
    c.q_len = q_len;
    c.q = (const char*)b->q + (size_t)q0 * b->q_stride_token * (b->dtype == ORACLE_F16 ? 2 : 4);
    c.q_stride_head = b->q_stride_head;
    c.q_stride_token = b->q_stride_token;
    c.kpool = b->key_pool;
    c.vpool = b->value_pool;
    /* The block table row holds the request's page_ids; only the pages that
       cover the length are handed over, as get_paged_cache_layout does. */
    for (int p = 0; p < npages; p++) ids[p] = b->block_tables[(size_t)s * b->max_pages_per_seq + p];
    c.page_ids = ids;
    c.num_page_ids = need < npages ? need : npages;
    c.page_count = b->num_pages;
    c.cached_token_count = L;
    float* scratch = (float*)malloc(sizeof(float) * (size_t)rep * q_len * L);
    float* vcat = (float*)malloc(sizeof(float) * (size_t)L * b->head_dim);
    double* y = (double*)malloc(sizeof(double) * (size_t)rep * q_len * b->head_dim);
    int rc = (!ids || !scratch || !vcat || !y) ? ORACLE_E_ALLOC : attend_group(&c, h, mode, y, scratch, vcat);
    if (rc == 0) {
      for (int r = 0; r < rep; r++)
        for (int i = 0; i < q_len; i++)
          for (int d = 0; d < b->head_dim; d++)
            out[((size_t)(h * rep + r) * total_q + q0 + i) * b->head_dim + d] =
                y[(size_t)(r * q_len + i) * b->head_dim + d];
    } else {
      rc_all |= 1;
    }
    free(ids);
    free(scratch);
    free(vcat);
    free(y);
  }
  return rc_all ? ORACLE_E_INVALID : 0;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
