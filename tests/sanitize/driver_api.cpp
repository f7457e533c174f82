// Sanitizer driver for the host half of libmvr_attn: argument checks,
// planning (workspace sizes over many shapes, with and without the host
// hints), the host-side table checks and the error paths of every entry
// point, built with AddressSanitizer and UndefinedBehaviorSanitizer on the
// host.  Nothing here launches a kernel: device pointers are aligned dummy
// addresses that only the device would dereference, and every call that
// would launch is made with arguments that fail first.  Host tables are
// heap arrays of exactly their documented sizes, so an out-of-bounds read by
// the planner or the validators is reported.  Exit status 0 on success.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "mvr_attn.h"

static int failures = 0;
#define CHECK(cond, ...)                                                                                               \
  do {                                                                                                                 \
    if (!(cond)) {                                                                                                     \
      fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);                                                              \
      fprintf(stderr, __VA_ARGS__);                                                                                    \
      fprintf(stderr, " (last error: %s)\n", mvr_last_error());                                                        \
      failures++;                                                                                                      \
    }                                                                                                                  \
  } while (0)

static void* fake(uintptr_t k) { return reinterpret_cast<void*>((uintptr_t)1 << 32 | (k << 12)); }

static mvr_paged_attention_args base_args(int dtype, int num_seqs, int hq, int hkv, int d, int page_size,
                                          int max_q_len, int max_seq_len) {
  mvr_paged_attention_args a;
  memset(&a, 0, sizeof a);
  a.dtype = dtype;
  a.num_seqs = num_seqs;
  a.num_q_heads = hq;
  a.num_kv_heads = hkv;
  a.head_dim = d;
  a.page_size = page_size;
  a.max_pages_per_seq = (max_seq_len + page_size - 1) / page_size;
  a.num_pages = (int64_t)num_seqs * a.max_pages_per_seq + 1;
  a.max_q_len = max_q_len;
  a.max_seq_len = max_seq_len;
  a.q = fake(1);
  a.key_pool = fake(2);
  a.value_pool = fake(3);
  a.block_tables = static_cast<const int32_t*>(fake(4));
  a.seq_lens = static_cast<const int32_t*>(fake(5));
  a.cu_q_lens = static_cast<const int32_t*>(fake(6));
  a.out = fake(7);
  const int64_t total_q = (int64_t)num_seqs * max_q_len;
  a.q_stride_head = a.out_stride_head = total_q * d;
  a.q_stride_token = a.out_stride_token = d;
  return a;
}

// Host tables of a batch: q_lens and cached lengths given; pages numbered in order.
struct Tables {
  std::vector<int32_t> bt, seq_lens, cu;
};

static Tables make_tables(const mvr_paged_attention_args& a, const std::vector<int>& q_lens,
                          const std::vector<int>& cached) {
  Tables t;
  t.bt.assign((size_t)a.num_seqs * a.max_pages_per_seq, 0);
  t.seq_lens.resize(a.num_seqs);
  t.cu.resize(a.num_seqs + 1);
  t.cu[0] = 0;
  int32_t next = 0;
  for (int s = 0; s < a.num_seqs; s++) {
    t.seq_lens[s] = cached[s] + q_lens[s];
    t.cu[s + 1] = t.cu[s] + q_lens[s];
    const int pages = (t.seq_lens[s] + a.page_size - 1) / a.page_size;
    for (int j = 0; j < pages; j++) t.bt[(size_t)s * a.max_pages_per_seq + j] = next++ % (int32_t)a.num_pages;
  }
  return t;
}

static void check_scalar_errors() {
  CHECK(mvr_paged_attention(nullptr) == MVR_E_INVALID_ARGUMENT, "null args");
  CHECK(mvr_paged_attention_workspace_size(nullptr) == 0, "null args size");
  struct Bad {
    const char* what;
    void (*edit)(mvr_paged_attention_args&);
  } bad[] = {
      {"dtype", [](mvr_paged_attention_args& a) { a.dtype = 7; }},
      {"head_dim", [](mvr_paged_attention_args& a) { a.head_dim = 80; }},
      {"heads", [](mvr_paged_attention_args& a) { a.num_q_heads = 30; }},
      {"page_size", [](mvr_paged_attention_args& a) { a.page_size = 0; }},
      {"num_seqs", [](mvr_paged_attention_args& a) { a.num_seqs = 0; }},
      {"max_q_len", [](mvr_paged_attention_args& a) { a.max_q_len = 0; }},
      {"pages", [](mvr_paged_attention_args& a) { a.max_pages_per_seq = 1; }},
      {"pool", [](mvr_paged_attention_args& a) { a.key_pool = nullptr; }},
      {"tables", [](mvr_paged_attention_args& a) { a.seq_lens = nullptr; }},
      {"align", [](mvr_paged_attention_args& a) { a.q = static_cast<const char*>(a.q) + 2; }},
  };
  for (const Bad& b : bad) {
    mvr_paged_attention_args a = base_args(MVR_DTYPE_F16, 4, 32, 8, 128, 16, 1, 1024);
    b.edit(a);
    CHECK(mvr_paged_attention(&a) != MVR_OK, "%s accepted", b.what);
    CHECK(mvr_last_error()[0] != 0, "%s: no error text", b.what);
    CHECK(mvr_paged_attention_noalloc(&a) != MVR_OK, "%s accepted by noalloc", b.what);
    CHECK(mvr_paged_attention_workspace_size(&a) == 0, "%s sized", b.what);
  }
}

// Workspace sizes over a grid of shapes, with and without each hint; the
// host hints are exact-size heap arrays read by the planner.
static void check_planning() {
  const int dtypes[] = {MVR_DTYPE_F32, MVR_DTYPE_F16};
  const int dims[] = {32, 64, 96, 128, 160, 256};
  const int pages[] = {16, 32, 48, 1, 2, 3, 5, 8, 24};
  struct Shape {
    int num_seqs, hq, hkv, max_q, max_seq;
  } shapes[] = {{1, 14, 2, 1, 512},  {8, 14, 2, 1, 4096},    {64, 32, 8, 1, 8192},
                {4, 28, 4, 256, 2304}, {16, 32, 8, 5, 16384}, {3, 8, 2, 17, 600}};
  size_t sized = 0;
  for (int dt : dtypes)
    for (int d : dims)
      for (int ps : pages)
        for (const Shape& sh : shapes) {
          mvr_paged_attention_args a = base_args(dt, sh.num_seqs, sh.hq, sh.hkv, d, ps, sh.max_q, sh.max_seq);
          (void)mvr_paged_attention_workspace_size(&a);
          std::vector<int> q_lens(sh.num_seqs), cached(sh.num_seqs);
          for (int s = 0; s < sh.num_seqs; s++) {
            q_lens[s] = s % 2 ? sh.max_q : 1 + (sh.max_q - 1) / 3;
            cached[s] = (sh.max_seq - q_lens[s]) * (s + 1) / sh.num_seqs;
          }
          Tables t = make_tables(a, q_lens, cached);
          int64_t sum = 0;
          for (int v : t.seq_lens) sum += v;
          a.sum_seq_lens = sum;
          (void)mvr_paged_attention_workspace_size(&a);
          a.total_q = t.cu.back(); // the plans guessed from the token count (no host tables)
          (void)mvr_paged_attention_workspace_size(&a);
          std::vector<int32_t> sl(t.seq_lens), cu(t.cu); // exact sizes: num_seqs and num_seqs + 1
          a.seq_lens_host = sl.data();
          a.cu_q_lens_host = cu.data();
          sized += mvr_paged_attention_workspace_size(&a) > 0;
          CHECK(mvr_paged_attention_validate(&a, t.bt.data(), t.seq_lens.data(), t.cu.data()) == MVR_OK,
                "valid tables rejected (D %d page %d seqs %d)", d, ps, sh.num_seqs);
        }
  CHECK(sized > 0, "no plan needed a workspace");

  // A scheduler step: 63 decodes at 8K and one 256-token chunk on a 2K prefix.
  mvr_paged_attention_args a = base_args(MVR_DTYPE_F16, 64, 32, 8, 128, 16, 256, 8192);
  std::vector<int> q_lens(64, 1), cached(64, 8191);
  q_lens[63] = 256;
  cached[63] = 2048;
  Tables t = make_tables(a, q_lens, cached);
  std::vector<int32_t> sl(t.seq_lens), cu(t.cu);
  a.seq_lens_host = sl.data();
  a.cu_q_lens_host = cu.data();
  CHECK(mvr_paged_attention_workspace_size(&a) > 0, "mixed batch sized 0");
  CHECK(mvr_paged_attention_validate(&a, t.bt.data(), sl.data(), cu.data()) == MVR_OK, "mixed tables rejected");
  // A hint that breaks the call's own bounds is not used (the plan falls back to one launch).
  cu[64] = cu[63] + 300;
  (void)mvr_paged_attention_workspace_size(&a);

  // The library's static scratch is bounded: a plan needing more is refused.
  for (int n = 256; n <= 16384; n *= 4) {
    mvr_paged_attention_args big = base_args(MVR_DTYPE_F32, n, 64, 8, 128, 16, 8, 32768);
    if (mvr_paged_attention_workspace_size(&big) > (size_t)MVR_NOALLOC_SCRATCH_BYTES) {
      CHECK(mvr_paged_attention_noalloc(&big) == MVR_E_WORKSPACE, "oversized noalloc call accepted");
      break;
    }
  }
}

static void check_validation_errors() {
  mvr_paged_attention_args a = base_args(MVR_DTYPE_F16, 3, 8, 2, 64, 16, 4, 200);
  Tables t = make_tables(a, {1, 4, 2}, {50, 0, 190});
  CHECK(mvr_paged_attention_validate(&a, t.bt.data(), t.seq_lens.data(), t.cu.data()) == MVR_OK, "valid rejected");
  {
    Tables u = t;
    u.bt[1 * a.max_pages_per_seq] = (int32_t)a.num_pages; // sequence 1's first page outside the pool
    CHECK(mvr_paged_attention_validate(&a, u.bt.data(), u.seq_lens.data(), u.cu.data()) == MVR_E_PAGE_ID, "page id");
  }
  {
    Tables u = t;
    u.seq_lens[2] = 1; // shorter than its q_len of 2
    CHECK(mvr_paged_attention_validate(&a, u.bt.data(), u.seq_lens.data(), u.cu.data()) != MVR_OK, "short seq_len");
  }
  {
    Tables u = t;
    u.seq_lens[0] = 201; // beyond max_seq_len
    CHECK(mvr_paged_attention_validate(&a, u.bt.data(), u.seq_lens.data(), u.cu.data()) != MVR_OK, "long seq_len");
  }
  {
    Tables u = t;
    u.cu[2] = u.cu[1]; // an empty request
    CHECK(mvr_paged_attention_validate(&a, u.bt.data(), u.seq_lens.data(), u.cu.data()) != MVR_OK, "empty request");
  }
  CHECK(mvr_paged_attention_validate(&a, nullptr, nullptr, nullptr) == MVR_OK, "no tables");
}

static void check_cascade() {
  mvr_paged_attention_args a = base_args(MVR_DTYPE_F16, 4, 8, 2, 128, 16, 2, 512);
  Tables t = make_tables(a, {1, 2, 1, 2}, {100, 64, 300, 200});
  // sequences 0-1 share their first 32 tokens (2 pages), sequence 2 is a group of one sharing nothing
  for (int j = 0; j < 2; j++) t.bt[1 * a.max_pages_per_seq + j] = t.bt[j];
  std::vector<int32_t> gcu = {0, 3, 4}, gpre = {32, 0}, spre = {32, 32, 0, 0};
  std::vector<int32_t> gbt(2 * (size_t)a.max_pages_per_seq, 0);
  for (int j = 0; j < a.max_pages_per_seq; j++) gbt[j] = t.bt[j];
  mvr_cascade_groups g;
  memset(&g, 0, sizeof g);
  g.num_groups = 2;
  g.max_group_q_len = 3;
  g.max_prefix_len = 32;
  g.group_cu_q_lens = static_cast<const int32_t*>(fake(8));
  g.group_prefix_lens = static_cast<const int32_t*>(fake(9));
  g.group_block_tables = static_cast<const int32_t*>(fake(10));
  g.seq_prefix_lens = static_cast<const int32_t*>(fake(11));
  CHECK(mvr_paged_attention_cascade_validate(&a, &g, t.bt.data(), t.seq_lens.data(), t.cu.data(), gcu.data(),
                                             gpre.data(), gbt.data(), spre.data()) == MVR_OK,
        "valid groups rejected");
  CHECK(mvr_paged_attention_cascade_workspace_size(&a, &g) > 0, "cascade sized 0");
  g.sum_prefix_lens = 64;
  a.sum_seq_lens = 673;
  (void)mvr_paged_attention_cascade_workspace_size(&a, &g); // the fallback rule's arithmetic
  std::vector<int32_t> bad_pre = {24, 0};                    // not a multiple of the page size
  CHECK(mvr_paged_attention_cascade_validate(&a, &g, t.bt.data(), t.seq_lens.data(), t.cu.data(), gcu.data(),
                                             bad_pre.data(), gbt.data(), spre.data()) != MVR_OK,
        "unaligned prefix accepted");
  g.num_groups = 5;
  CHECK(mvr_paged_attention_cascade(&a, &g) == MVR_E_INVALID_ARGUMENT, "too many groups accepted");
}

static void check_request_level() {
  mvr_attention_dimensions dims = {14, 2, 64, 500, 1};
  mvr_paged_cache_layout lay;
  memset(&lay, 0, sizeof lay);
  lay.key_pool = fake(12);
  lay.value_pool = fake(13);
  lay.page_count = 64;
  lay.page_ids = static_cast<const int32_t*>(fake(14));
  lay.num_page_ids = 32;
  lay.per_page_token_count = 16;
  lay.cached_token_count = 501;
  (void)mvr_forward_paged_attention_workspace_size(MVR_DTYPE_F32, &dims, &lay);
  lay.cached_token_count = 502; // the reference's length check
  CHECK(mvr_forward_paged_attention(MVR_DTYPE_F32, &dims, &lay, fake(15), fake(16), nullptr, 0, nullptr) ==
            MVR_E_LENGTH_MISMATCH,
        "length mismatch accepted");
  lay.cached_token_count = 501;
  lay.num_page_ids = 31; // 496 tokens of pages for 501
  CHECK(mvr_forward_paged_attention(MVR_DTYPE_F32, &dims, &lay, fake(15), fake(16), nullptr, 0, nullptr) ==
            MVR_E_PAGES_UNCOVERED,
        "uncovered pages accepted");
  CHECK(mvr_reconstruct_contiguous(MVR_DTYPE_F16, fake(17), 64, 2, 16, 64, static_cast<const int32_t*>(fake(18)), 0,
                                   0, fake(19), nullptr) != MVR_OK,
        "empty reconstruct accepted");
}

static void check_rope_append() {
  mvr_rope_append_args r;
  memset(&r, 0, sizeof r);
  r.dtype = MVR_DTYPE_F16;
  r.rope_type = MVR_ROPE_NEOX;
  r.num_seqs = 2;
  r.num_q_heads = 8;
  r.num_kv_heads = 2;
  r.head_dim = 64;
  r.page_size = 16;
  r.max_pages_per_seq = 8;
  r.num_pages = 16;
  r.total_q = 5;
  r.max_seq_len = 100;
  r.rope_len = 128;
  r.q = r.q_out = fake(20);
  r.k = fake(21);
  r.v = fake(22);
  r.cos_table = fake(23);
  r.sin_table = fake(24);
  r.block_tables = static_cast<const int32_t*>(fake(25));
  r.seq_lens = static_cast<const int32_t*>(fake(26));
  r.cu_q_lens = static_cast<const int32_t*>(fake(27));
  r.key_pool = fake(28);
  r.value_pool = fake(29);
  r.q_stride_head = r.q_out_stride_head = 5 * 64;
  r.k_stride_head = r.v_stride_head = 5 * 64;
  r.q_stride_token = r.q_out_stride_token = r.k_stride_token = r.v_stride_token = 64;
  std::vector<int32_t> bt(16), sl = {40, 100}, cu = {0, 1, 5};
  for (int i = 0; i < 16; i++) bt[i] = i;
  std::vector<uint8_t> writable(16, 1);
  CHECK(mvr_rope_append_validate(&r, bt.data(), sl.data(), cu.data(), writable.data()) == MVR_OK, "valid append");
  writable[2] = 0; // sequence 0 writes position 39, page 2
  CHECK(mvr_rope_append_validate(&r, bt.data(), sl.data(), cu.data(), writable.data()) == MVR_E_READ_ONLY_PAGE,
        "read-only page");
  std::vector<int32_t> cu_empty = {0, 0, 5};
  CHECK(mvr_rope_append_validate(&r, bt.data(), sl.data(), cu_empty.data(), nullptr) != MVR_OK, "empty append");
  std::vector<int32_t> bt_shared(bt);
  bt_shared[8 + 6] = bt_shared[2]; // sequence 1 writes a page sequence 0 writes too
  CHECK(mvr_rope_append_validate(&r, bt_shared.data(), sl.data(), cu.data(), nullptr) != MVR_OK, "shared page");
  mvr_rope_append_args bad = r;
  bad.rope_type = 5;
  CHECK(mvr_rope_append(&bad) == MVR_E_UNSUPPORTED, "rope type");
  bad = r;
  bad.rope_len = 50;
  CHECK(mvr_rope_append(&bad) == MVR_E_INVALID_ARGUMENT, "short rotary tables");
  CHECK(mvr_rope_append(nullptr) == MVR_E_INVALID_ARGUMENT, "null rope args");
}

int main() {
  CHECK(mvr_abi_version() == MVR_ATTN_ABI_VERSION, "ABI version %d", mvr_abi_version());
  check_scalar_errors();
  check_planning();
  check_validation_errors();
  check_cascade();
  check_request_level();
  check_rope_append();
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("library host sanitizer driver: all checks passed\n");
  return 0;
}
