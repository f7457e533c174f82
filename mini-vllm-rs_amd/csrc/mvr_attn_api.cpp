// C ABI of libmvr_attn.so: argument checks, grid planning, workspace sizing
// and dispatch to the HIP kernels.  Declared in include/mvr_attn.h.
#include "mvr_attn.h"

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "paged_attention_kernels.hpp"

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

// Read-once environment overrides, in the reference's idiom of LazyLock flags
// (src/models/backends/common.rs:28-58, src/utils/mod.rs:5-23).
int env_int(const char* name, int fallback) {
  const char* v = getenv(name);
  if (!v || !*v) return fallback;
  char* end = nullptr;
  long x = strtol(v, &end, 10);
  return (end && *end == 0 && x > 0 && x < (1L << 30)) ? (int)x : fallback;
}

int chunks_per_partition_override() {
  static const int v = env_int("MVR_ATTN_CHUNKS_PER_PARTITION", 0);
  return v;
}

int target_waves_override() {
  static const int v = env_int("MVR_ATTN_TARGET_WAVES", 0);
  return v;
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Scalar checks shared by every entry point.
int check_scalars(const mvr_paged_attention_args* a) {
  if (!a) return fail(MVR_E_INVALID_ARGUMENT, "args is null");
  if (a->dtype != MVR_DTYPE_F32 && a->dtype != MVR_DTYPE_F16)
    return fail(MVR_E_UNSUPPORTED, "dtype %d is not F32 (0) or F16 (1)", a->dtype);
  if (a->num_seqs < 1) return fail(MVR_E_INVALID_ARGUMENT, "forward requires at least one request");
  if (a->num_kv_heads < 1 || a->num_q_heads < 1 || a->num_q_heads % a->num_kv_heads != 0)
    return fail(MVR_E_INVALID_ARGUMENT, "num_q_heads %d is not a multiple of num_kv_heads %d", a->num_q_heads,
                a->num_kv_heads);
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(MVR_E_UNSUPPORTED, "head_dim %d is not supported (64 or 128)", a->head_dim);
  if (a->page_size < mvr::kChunkTokens || a->page_size % mvr::kChunkTokens != 0)
    return fail(MVR_E_UNSUPPORTED, "page_size %d is not a positive multiple of %d", a->page_size,
                mvr::kChunkTokens);
  if (a->num_pages < 1) return fail(MVR_E_INVALID_ARGUMENT, "num_pages must be positive");
  if (a->max_q_len < 1) return fail(MVR_E_INVALID_ARGUMENT, "each forward input must contain at least one token");
  if (a->max_seq_len < a->max_q_len)
    return fail(MVR_E_INVALID_ARGUMENT, "max_seq_len %d is smaller than max_q_len %d", a->max_seq_len, a->max_q_len);
  const int64_t pages_needed = (a->max_seq_len + a->page_size - 1) / a->page_size;
  if (a->max_pages_per_seq < pages_needed)
    return fail(MVR_E_PAGES_UNCOVERED,
                "paged KV cache contains fewer pages than its sequence length, leaving %lld tokens uncovered",
                (long long)(a->max_seq_len - (int64_t)a->max_pages_per_seq * a->page_size));
  if (a->num_seqs > 1 && (!a->seq_lens || !a->cu_q_lens))
    return fail(MVR_E_INVALID_ARGUMENT, "seq_lens and cu_q_lens are required when num_seqs > 1");
  if (!a->q || !a->key_pool || !a->value_pool || !a->block_tables || !a->out)
    return fail(MVR_E_INVALID_ARGUMENT, "null q, pool, block table or output pointer");
  const int64_t vec = a->dtype == MVR_DTYPE_F16 ? 8 : 4; // elements per 16-byte access
  if (!aligned16(a->q) || !aligned16(a->out) || !aligned16(a->key_pool) || !aligned16(a->value_pool) ||
      a->q_stride_head % vec || a->q_stride_token % vec || a->out_stride_head % vec || a->out_stride_token % vec)
    return fail(MVR_E_INVALID_ARGUMENT, "q, out and pools must be 16-byte aligned with strides multiple of %lld",
                (long long)vec);
  if (a->scale < 0.f || !isfinite(a->scale)) return fail(MVR_E_INVALID_ARGUMENT, "scale must be finite and >= 0");
  return MVR_OK;
}

mvr::PagedAttentionPlan make_plan(const mvr_paged_attention_args* a) {
  mvr::PagedAttentionPlan plan{};
  plan.dtype = a->dtype;
  plan.head_dim = a->head_dim;
  const int group = a->num_q_heads / a->num_kv_heads;
  const int64_t rows_max = (int64_t)group * a->max_q_len;
  plan.row_blocks = rows_max <= 16 ? 1 : 2;
  const int tile_rows = 16 * plan.row_blocks;
  plan.row_tiles = (int)((rows_max + tile_rows - 1) / tile_rows);
  const int max_chunks = (a->max_seq_len + mvr::kChunkTokens - 1) / mvr::kChunkTokens;
  const int64_t base_units = (int64_t)a->num_seqs * a->num_kv_heads * plan.row_tiles;
  int cpp = chunks_per_partition_override();
  if (cpp <= 0) {
    // Split contexts so that the units fill the resident wavefront slots of
    // the device once: more partitions add merge traffic and a tail round,
    // fewer leave CUs idle.
    int64_t slots = target_waves_override();
    if (slots <= 0) slots = mvr::paged_attention_resident_waves(plan.dtype, plan.head_dim, plan.row_blocks);
    if (slots <= 0) slots = 256 * 8; // no device to ask (sizing only)
    int64_t parts = slots / base_units;
    if (parts < 1) parts = 1;
    cpp = (int)((max_chunks + parts - 1) / parts);
    if (cpp < 8) cpp = 8; // at least 128 tokens per wavefront
  }
  if (cpp > max_chunks) cpp = max_chunks;
  plan.chunks_per_part = cpp;
  plan.max_parts = (max_chunks + cpp - 1) / cpp;
  plan.num_units = base_units * plan.max_parts;
  plan.partial_bytes = 0;
  if (plan.max_parts > 1) {
    // [partial o][partial m, l]
    const size_t prow = (size_t)plan.num_units * tile_rows;
    plan.partial_bytes = align_up(prow * a->head_dim * sizeof(float), 256) + align_up(prow * 2 * sizeof(float), 256);
  }
  return plan;
}

} // namespace

extern "C" {

int mvr_abi_version(void) { return MVR_ATTN_ABI_VERSION; }

const char* mvr_last_error(void) { return g_last_error; }

size_t mvr_paged_attention_workspace_size(const mvr_paged_attention_args* args) {
  if (check_scalars(args) != MVR_OK) return 0;
  return make_plan(args).partial_bytes;
}

int mvr_paged_attention(const mvr_paged_attention_args* a) {
  g_last_error[0] = 0;
  int rc = check_scalars(a);
  if (rc != MVR_OK) return rc;
  const mvr::PagedAttentionPlan plan = make_plan(a);
  if (a->workspace_bytes < plan.partial_bytes || (plan.partial_bytes && !a->workspace))
    return fail(MVR_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", a->workspace_bytes,
                plan.partial_bytes);
  if (plan.partial_bytes && ((uintptr_t)a->workspace & 255u))
    return fail(MVR_E_INVALID_ARGUMENT, "workspace must be 256-byte aligned");

  mvr::PagedAttentionParams p{};
  p.q = a->q;
  p.q_stride_head = a->q_stride_head;
  p.q_stride_token = a->q_stride_token;
  p.key_pool = a->key_pool;
  p.value_pool = a->value_pool;
  p.block_tables = a->block_tables;
  p.block_table_stride = a->max_pages_per_seq;
  p.seq_lens = a->seq_lens;
  p.cu_q_lens = a->cu_q_lens;
  p.single_seq_len = a->max_seq_len;
  p.single_q_len = a->max_q_len;
  p.out = a->out;
  p.out_stride_head = a->out_stride_head;
  p.out_stride_token = a->out_stride_token;
  if (plan.partial_bytes) {
    const size_t prow = (size_t)plan.num_units * 16 * plan.row_blocks;
    char* ws = static_cast<char*>(a->workspace);
    p.partial_o = reinterpret_cast<float*>(ws);
    p.partial_ml = reinterpret_cast<float*>(ws + align_up(prow * a->head_dim * sizeof(float), 256));
  }
  p.num_seqs = a->num_seqs;
  p.num_kv_heads = a->num_kv_heads;
  p.group_size = a->num_q_heads / a->num_kv_heads;
  p.page_size = a->page_size;
  const float scale = a->scale > 0.f ? a->scale : (float)(1.0 / sqrt((double)a->head_dim));
  p.scale_log2 = scale * 1.4426950408889634f;

  hipError_t err = mvr::launch_paged_attention(plan, p, static_cast<hipStream_t>(a->stream));
  if (err != hipSuccess) return fail(MVR_E_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return MVR_OK;
}

int mvr_paged_attention_validate(const mvr_paged_attention_args* a, const int32_t* block_tables_host,
                                 const int32_t* seq_lens_host, const int32_t* cu_q_lens_host) {
  g_last_error[0] = 0;
  int rc = check_scalars(a);
  if (rc != MVR_OK) return rc;
  for (int s = 0; s < a->num_seqs; s++) {
    const int seq_len = seq_lens_host ? seq_lens_host[s] : (a->num_seqs == 1 ? a->max_seq_len : -1);
    int q_len = -1;
    if (cu_q_lens_host) {
      if (s == 0 && cu_q_lens_host[0] != 0) return fail(MVR_E_INVALID_ARGUMENT, "cu_q_lens[0] must be 0");
      q_len = cu_q_lens_host[s + 1] - cu_q_lens_host[s];
    } else if (a->num_seqs == 1) {
      q_len = a->max_q_len;
    }
    if (q_len >= 0) {
      if (q_len < 1) return fail(MVR_E_INVALID_ARGUMENT, "each forward input must contain at least one token");
      if (q_len > a->max_q_len) return fail(MVR_E_INVALID_ARGUMENT, "request %d has q_len %d > max_q_len %d", s, q_len, a->max_q_len);
    }
    if (seq_len >= 0) {
      if (seq_len > a->max_seq_len)
        return fail(MVR_E_INVALID_ARGUMENT, "request %d has seq_len %d > max_seq_len %d", s, seq_len, a->max_seq_len);
      if (q_len >= 0 && seq_len < q_len)
        // cached_token_count must equal cached_kv_len + q_len with cached_kv_len >= 0 (common.rs:447-454)
        return fail(MVR_E_LENGTH_MISMATCH, "paged KV cache reports sequence length %d, expected at least %d", seq_len,
                    q_len);
      if (block_tables_host) {
        const int need = (seq_len + a->page_size - 1) / a->page_size;
        for (int pi = 0; pi < need; pi++) {
          const int32_t id = block_tables_host[(int64_t)s * a->max_pages_per_seq + pi];
          if (id < 0 || id >= a->num_pages)
            return fail(MVR_E_PAGE_ID, "request %d page %d has id %d outside a pool of %lld pages", s, pi, id,
                        (long long)a->num_pages);
        }
      }
    }
  }
  return MVR_OK;
}

static int layout_to_args(int32_t dtype, const mvr_attention_dimensions* dims, const mvr_paged_cache_layout* layout,
                          const void* request_q, void* request_y, void* workspace, size_t workspace_bytes, void* stream,
                          mvr_paged_attention_args* a) {
  if (!dims || !layout) return fail(MVR_E_INVALID_ARGUMENT, "dims or layout is null");
  const int64_t expected = (int64_t)dims->cached_kv_len + dims->q_len;
  if (layout->cached_token_count != expected) // common.rs:447-454
    return fail(MVR_E_LENGTH_MISMATCH, "paged KV cache reports sequence length %d, expected %lld",
                layout->cached_token_count, (long long)expected);
  if (layout->per_page_token_count > 0) {
    const int64_t covered = (int64_t)layout->num_page_ids * layout->per_page_token_count;
    if (covered < layout->cached_token_count) // common.rs:776-781
      return fail(MVR_E_PAGES_UNCOVERED,
                  "paged KV cache contains fewer pages than its sequence length, leaving %lld tokens uncovered",
                  (long long)(layout->cached_token_count - covered));
  }
  memset(a, 0, sizeof(*a));
  a->dtype = dtype;
  a->num_seqs = 1;
  a->num_q_heads = dims->num_q_heads;
  a->num_kv_heads = dims->num_kv_heads;
  a->head_dim = dims->head_dim;
  a->page_size = layout->per_page_token_count;
  a->num_pages = layout->page_count;
  a->max_pages_per_seq = layout->num_page_ids;
  a->max_q_len = dims->q_len;
  a->max_seq_len = layout->cached_token_count;
  a->q = request_q; // [1, Hq, q_len, D]
  a->q_stride_head = (int64_t)dims->q_len * dims->head_dim;
  a->q_stride_token = dims->head_dim;
  a->key_pool = layout->key_pool;
  a->value_pool = layout->value_pool;
  a->block_tables = layout->page_ids;
  a->out = request_y;
  a->out_stride_head = (int64_t)dims->q_len * dims->head_dim;
  a->out_stride_token = dims->head_dim;
  a->workspace = workspace;
  a->workspace_bytes = workspace_bytes;
  a->stream = stream;
  return MVR_OK;
}

int mvr_forward_paged_attention(int32_t dtype, const mvr_attention_dimensions* dims,
                                const mvr_paged_cache_layout* layout, const void* request_q, void* request_y,
                                void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error[0] = 0;
  mvr_paged_attention_args a;
  int rc = layout_to_args(dtype, dims, layout, request_q, request_y, workspace, workspace_bytes, stream, &a);
  if (rc != MVR_OK) return rc;
  return mvr_paged_attention(&a);
}

size_t mvr_forward_paged_attention_workspace_size(int32_t dtype, const mvr_attention_dimensions* dims,
                                                  const mvr_paged_cache_layout* layout) {
  mvr_paged_attention_args a;
  if (layout_to_args(dtype, dims, layout, nullptr, nullptr, nullptr, 0, nullptr, &a) != MVR_OK) return 0;
  a.q = a.out = reinterpret_cast<void*>(256); // scalar sizing only
  if (!a.key_pool) a.key_pool = a.q;
  if (!a.value_pool) a.value_pool = a.q;
  if (!a.block_tables) a.block_tables = reinterpret_cast<const int32_t*>(256);
  return mvr_paged_attention_workspace_size(&a);
}

} // extern "C"
