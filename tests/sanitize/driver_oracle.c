/*
 * Sanitizer driver for the oracle (test infrastructure): runs every oracle
 * entry point over seeded inputs held in exactly sized heap buffers, so that
 * AddressSanitizer catches any read or write outside them and
 * UndefinedBehaviorSanitizer any undefined arithmetic.  Also checks the
 * documented error codes of malformed requests and that results are finite.
 * Exit status 0 on success.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kv_append_oracle.h"
#include "paged_attention_oracle.h"

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;

static uint32_t rnd(void) {
  rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(rng_state >> 33);
}

static float rnd_val(void) { return ((float)(rnd() % 2001) - 1000.f) / 1000.f; }

static void* xmalloc(size_t n) {
  void* p = malloc(n ? n : 1);
  if (!p) {
    fprintf(stderr, "out of memory\n");
    exit(2);
  }
  return p;
}

static size_t elem_size(int dtype) { return dtype == ORACLE_F16 ? 2 : 4; }

static void fill(void* buf, size_t n, int dtype) {
  for (size_t i = 0; i < n; i++) {
    const float v = rnd_val();
    if (dtype == ORACLE_F16)
      ((uint16_t*)buf)[i] = oracle_f32_to_f16(v);
    else
      ((float*)buf)[i] = v;
  }
}

static int failures = 0;
#define CHECK(cond, ...)                                                                                               \
  do {                                                                                                                 \
    if (!(cond)) {                                                                                                     \
      fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);                                                              \
      fprintf(stderr, __VA_ARGS__);                                                                                    \
      fprintf(stderr, "\n");                                                                                           \
      failures++;                                                                                                      \
    }                                                                                                                  \
  } while (0)

/* A packed batch with q_lens[s] new tokens after cached[s] cached ones, pages
   scattered over a pool with a few spare pages. */
static void run_batch(int dtype, int hq, int hkv, int d, int page_size, int num_seqs, const int* q_lens,
                      const int* cached, int mode, int threads) {
  int32_t* seq_lens = xmalloc(sizeof(int32_t) * num_seqs);
  int32_t* cu = xmalloc(sizeof(int32_t) * (num_seqs + 1));
  int max_pages = 0;
  int64_t total_pages = 0;
  cu[0] = 0;
  for (int s = 0; s < num_seqs; s++) {
    seq_lens[s] = cached[s] + q_lens[s];
    cu[s + 1] = cu[s] + q_lens[s];
    const int pages = (seq_lens[s] + page_size - 1) / page_size;
    if (pages > max_pages) max_pages = pages;
    total_pages += pages;
  }
  const int64_t num_pages = total_pages + 3;
  int32_t* bt = xmalloc(sizeof(int32_t) * (size_t)num_seqs * max_pages);
  int64_t next = 0;
  for (int s = 0; s < num_seqs; s++)
    for (int j = 0; j < max_pages; j++)
      bt[(size_t)s * max_pages + j] = j < (seq_lens[s] + page_size - 1) / page_size ? (int32_t)((next++ * 7 + 3) % num_pages) : 0;
  const int total_q = cu[num_seqs];
  const size_t es = elem_size(dtype);
  const size_t pool_elems = (size_t)num_pages * hkv * page_size * d;
  void* q = xmalloc(es * (size_t)hq * total_q * d);
  void* kp = xmalloc(es * pool_elems);
  void* vp = xmalloc(es * pool_elems);
  fill(q, (size_t)hq * total_q * d, dtype);
  fill(kp, pool_elems, dtype);
  fill(vp, pool_elems, dtype);
  double* out = xmalloc(sizeof(double) * (size_t)hq * total_q * d);
  oracle_batch b;
  memset(&b, 0, sizeof b);
  b.dtype = dtype;
  b.num_seqs = num_seqs;
  b.num_q_heads = hq;
  b.num_kv_heads = hkv;
  b.head_dim = d;
  b.page_size = page_size;
  b.num_pages = num_pages;
  b.max_pages_per_seq = max_pages;
  b.q = q;
  b.q_stride_head = (int64_t)total_q * d;
  b.q_stride_token = d;
  b.key_pool = kp;
  b.value_pool = vp;
  b.block_tables = bt;
  b.seq_lens = seq_lens;
  b.cu_q_lens = cu;
  const int rc = oracle_paged_attention(&b, mode, threads, out);
  CHECK(rc == ORACLE_OK, "oracle_paged_attention rc %d (dtype %d D %d page %d mode %d)", rc, dtype, d, page_size, mode);
  for (size_t i = 0; i < (size_t)hq * total_q * d; i++)
    if (!isfinite(out[i])) {
      CHECK(0, "non-finite output at %zu", i);
      break;
    }

  /* The single-request entry points on sequence 0, and their error codes. */
  const int L = seq_lens[0];
  const int npg = (L + page_size - 1) / page_size;
  int64_t* ids = xmalloc(sizeof(int64_t) * npg);
  for (int j = 0; j < npg; j++) ids[j] = bt[j];
  oracle_dims dims = {dtype, hq, hkv, d, cached[0], q_lens[0]};
  const int ql = q_lens[0];
  void* rq = xmalloc(es * (size_t)hq * ql * d);
  fill(rq, (size_t)hq * ql * d, dtype);
  double* ry = xmalloc(sizeof(double) * (size_t)hq * ql * d);
  char err[256];
  int r = oracle_forward_paged_attention(&dims, rq, kp, vp, num_pages, ids, npg, page_size, L, mode, ry, err, sizeof err);
  CHECK(r == ORACLE_OK, "forward_paged_attention rc %d: %s", r, err);
  r = oracle_forward_paged_attention(&dims, rq, kp, vp, num_pages, ids, npg, page_size, L + 1, mode, ry, err, sizeof err);
  CHECK(r == ORACLE_E_LENGTH, "length mismatch gave %d", r);
  if (npg > 1) {
    r = oracle_forward_paged_attention(&dims, rq, kp, vp, num_pages, ids, npg - 1, page_size, L, mode, ry, err,
                                       sizeof err);
    CHECK(r == ORACLE_E_UNCOVERED, "uncovered pages gave %d", r);
  }
  const int64_t saved = ids[0];
  ids[0] = num_pages;
  r = oracle_forward_paged_attention(&dims, rq, kp, vp, num_pages, ids, npg, page_size, L, mode, ry, err, sizeof err);
  CHECK(r == ORACLE_E_PAGE_ID, "page id outside the pool gave %d", r);
  ids[0] = saved;

  /* Gather to contiguous K and the contiguous attention over it. */
  void* kc = xmalloc(es * (size_t)hkv * L * d);
  void* vc = xmalloc(es * (size_t)hkv * L * d);
  r = oracle_reconstruct_contiguous(dtype, kp, hkv, page_size, d, num_pages, ids, npg, L, kc);
  CHECK(r == ORACLE_OK, "reconstruct K rc %d", r);
  r = oracle_reconstruct_contiguous(dtype, vp, hkv, page_size, d, num_pages, ids, npg, L, vc);
  CHECK(r == ORACLE_OK, "reconstruct V rc %d", r);
  r = oracle_forward_contiguous_attention(&dims, rq, kc, vc, L, mode, ry);
  CHECK(r == ORACLE_OK, "contiguous attention rc %d", r);

  free(kc);
  free(vc);
  free(ry);
  free(rq);
  free(ids);
  free(out);
  free(q);
  free(kp);
  free(vp);
  free(bt);
  free(cu);
  free(seq_lens);
}

/* RoPE + append of a packed batch, then the error paths of one request. */
static void run_rope_append(int dtype, int rope_type, int d, int page_size) {
  enum { S = 3, HQ = 4, HKV = 2 };
  const int q_lens[S] = {1, 6, 3};
  const int cached[S] = {20, 0, 33};
  int32_t seq_lens[S], cu[S + 1];
  cu[0] = 0;
  int max_pages = 0, rope_len = 0;
  for (int s = 0; s < S; s++) {
    seq_lens[s] = cached[s] + q_lens[s];
    cu[s + 1] = cu[s] + q_lens[s];
    const int p = (seq_lens[s] + page_size - 1) / page_size;
    if (p > max_pages) max_pages = p;
    if (seq_lens[s] > rope_len) rope_len = seq_lens[s];
  }
  const int64_t num_pages = (int64_t)S * max_pages + 2;
  int32_t* bt = xmalloc(sizeof(int32_t) * S * max_pages);
  for (int i = 0; i < S * max_pages; i++) bt[i] = (int32_t)((i * 5 + 1) % num_pages);
  const int total_q = cu[S];
  const size_t es = elem_size(dtype);
  void* q = xmalloc(es * (size_t)HQ * total_q * d);
  void* k = xmalloc(es * (size_t)HKV * total_q * d);
  void* v = xmalloc(es * (size_t)HKV * total_q * d);
  void* qo = xmalloc(es * (size_t)HQ * total_q * d);
  void* cosv = xmalloc(es * (size_t)rope_len * (d / 2));
  void* sinv = xmalloc(es * (size_t)rope_len * (d / 2));
  const size_t pool_elems = (size_t)num_pages * HKV * page_size * d;
  void* kp = xmalloc(es * pool_elems);
  void* vp = xmalloc(es * pool_elems);
  fill(q, (size_t)HQ * total_q * d, dtype);
  fill(k, (size_t)HKV * total_q * d, dtype);
  fill(v, (size_t)HKV * total_q * d, dtype);
  fill(cosv, (size_t)rope_len * (d / 2), dtype);
  fill(sinv, (size_t)rope_len * (d / 2), dtype);
  memset(kp, 0, es * pool_elems);
  memset(vp, 0, es * pool_elems);
  oracle_rope_append_batch b;
  memset(&b, 0, sizeof b);
  b.dtype = dtype;
  b.rope_type = rope_type;
  b.num_seqs = S;
  b.num_q_heads = HQ;
  b.num_kv_heads = HKV;
  b.head_dim = d;
  b.page_size = page_size;
  b.num_pages = num_pages;
  b.max_pages_per_seq = max_pages;
  b.q = q;
  b.q_stride_head = (int64_t)total_q * d;
  b.q_stride_token = d;
  b.k = k;
  b.k_stride_head = (int64_t)total_q * d;
  b.k_stride_token = d;
  b.v = v;
  b.v_stride_head = (int64_t)total_q * d;
  b.v_stride_token = d;
  b.cos_table = cosv;
  b.sin_table = sinv;
  b.rope_len = rope_len;
  b.block_tables = bt;
  b.seq_lens = seq_lens;
  b.cu_q_lens = cu;
  b.q_out = qo;
  b.q_out_stride_head = (int64_t)total_q * d;
  b.q_out_stride_token = d;
  b.key_pool = kp;
  b.value_pool = vp;
  char err[256];
  int r = oracle_rope_append(&b, err, sizeof err);
  CHECK(r == ORACLE_APPEND_OK, "rope_append rc %d: %s", r, err);
  b.rope_len = rope_len - 1; /* the last position has no rotary row */
  r = oracle_rope_append(&b, err, sizeof err);
  CHECK(r == ORACLE_APPEND_E_ROPE_RANGE, "short rotary tables gave %d", r);

  /* RoPE alone, in the dtype and in double. */
  double* xd = xmalloc(sizeof(double) * (size_t)HQ * 3 * d);
  double* yd = xmalloc(sizeof(double) * (size_t)HQ * 3 * d);
  double* cd = xmalloc(sizeof(double) * (size_t)rope_len * (d / 2));
  double* sd = xmalloc(sizeof(double) * (size_t)rope_len * (d / 2));
  for (size_t i = 0; i < (size_t)HQ * 3 * d; i++) xd[i] = rnd_val();
  for (size_t i = 0; i < (size_t)rope_len * (d / 2); i++) {
    cd[i] = rnd_val();
    sd[i] = rnd_val();
  }
  r = oracle_rope_f64(rope_type, xd, HQ, 3, d, cd, sd, rope_len, rope_len - 3, yd);
  CHECK(r == 0, "rope_f64 rc %d", r);
  r = oracle_rope(dtype, rope_type, q, HQ, 3, d, cosv, sinv, rope_len, rope_len - 3, qo);
  CHECK(r == 0, "rope rc %d", r);

  /* append_pages: a read-only page and a missing page are refused. */
  int64_t ids[4] = {0, 1, 2, 3};
  uint8_t* writable = xmalloc((size_t)num_pages);
  memset(writable, 1, (size_t)num_pages);
  const int tokens = 2;
  void* kk = xmalloc(es * (size_t)HKV * tokens * d);
  void* vv = xmalloc(es * (size_t)HKV * tokens * d);
  fill(kk, (size_t)HKV * tokens * d, dtype);
  fill(vv, (size_t)HKV * tokens * d, dtype);
  r = oracle_append_pages(es, kp, vp, num_pages, HKV, page_size, d, ids, 4, page_size - 1, kk, vv, tokens, writable,
                          err, sizeof err);
  CHECK(r == ORACLE_APPEND_OK, "append_pages rc %d: %s", r, err);
  writable[1] = 0;
  r = oracle_append_pages(es, kp, vp, num_pages, HKV, page_size, d, ids, 4, page_size - 1, kk, vv, tokens, writable,
                          err, sizeof err);
  CHECK(r == ORACLE_APPEND_E_READ_ONLY, "read-only page gave %d", r);
  r = oracle_append_pages(es, kp, vp, num_pages, HKV, page_size, d, ids, 1, page_size - 1, kk, vv, tokens, NULL, err,
                          sizeof err);
  CHECK(r == ORACLE_APPEND_E_MISSING, "missing page gave %d", r);
  r = oracle_append_pages(es, kp, vp, num_pages, HKV, page_size, d, ids, 4, 0, kk, vv, 0, NULL, err, sizeof err);
  CHECK(r == ORACLE_APPEND_E_EMPTY, "empty append gave %d", r);

  free(kk);
  free(vv);
  free(writable);
  free(xd);
  free(yd);
  free(cd);
  free(sd);
  free(q);
  free(k);
  free(v);
  free(qo);
  free(cosv);
  free(sinv);
  free(kp);
  free(vp);
  free(bt);
}

int main(void) {
  const int dec_q[4] = {1, 1, 1, 1}, dec_c[4] = {511, 37, 1, 260};
  const int mix_q[3] = {1, 17, 5}, mix_c[3] = {300, 0, 64};
  const int dts[2] = {ORACLE_F32, ORACLE_F16};
  const int dims[2] = {64, 128};
  for (int t = 0; t < 2; t++)
    for (int di = 0; di < 2; di++) {
      const int dt = dts[t], d = dims[di];
      run_batch(dt, 14, 2, d, 16, 4, dec_q, dec_c, ORACLE_REF_CONCAT_V, 1);
      run_batch(dt, 8, 2, d, 5, 3, mix_q, mix_c, ORACLE_REF_PAGEWISE_V, 4);
      run_batch(dt, 32, 8, d, 32, 3, mix_q, mix_c, ORACLE_EXACT_F64, 2);
      run_rope_append(dt, ORACLE_ROPE_NEOX, d, 16);
      run_rope_append(dt, ORACLE_ROPE_INTERLEAVED, d, 3);
    }
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("oracle sanitizer driver: all checks passed\n");
  return 0;
}
