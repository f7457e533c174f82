// C ABI of libmvr_attn.so: argument checks, grid planning, workspace sizing
// and dispatch to the HIP kernels.  Declared in include/mvr_attn.h.
#include "mvr_attn.h"

#include <hip/hip_runtime.h>
#include <rocprofiler-sdk-roctx/roctx.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "kv_append.hpp"
#include "kv_gather.hpp"
#include "paged_attention_kernels.hpp"
#include "paged_prefill.hpp"

// Device scratch of mvr_paged_attention_noalloc (split-context partials and
// the 16-token repack), one copy per device from module load until the
// process ends.  In host code `scratch` names a host-side stand-in, never
// the device array: its device address comes from hipGetSymbolAddress
// (noalloc_scratch below), once per device.
static __device__ __align__(256) unsigned char scratch[MVR_NOALLOC_SCRATCH_BYTES];

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

// "true" / "false" as Rust's bool parser accepts them (src/utils/mod.rs:5-13);
// anything else keeps the default instead of aborting the host process.
bool env_bool(const char* name, bool fallback) {
  const char* v = getenv(name);
  if (!v) return fallback;
  if (strcmp(v, "true") == 0) return true;
  if (strcmp(v, "false") == 0) return false;
  return fallback;
}

// roctx ranges named like the reference's tracing spans (trace.rs:64-116,
// mirrored to NVTX by nvtx_trace.rs:14-53, whose labels are the span name
// followed by its fields as " field=value"), on when MVR_ENABLE_ROCTX=true.
bool roctx_enabled() {
  static const bool v = env_bool("MVR_ENABLE_ROCTX", false);
  return v;
}

// Development mode, on when MVR_ATTN_CHECKED=true: every call copies the
// device tables it is about to trust back to the host (stream-ordered, then
// waits for the stream) and runs the host checks of the matching *_validate
// entry point first, so that tables breaking the contract come back as an
// MVR_E_* error instead of wrong reads.  It synchronises the stream and
// allocates host memory on every call: not for serving.
bool checked_mode() {
  static const bool v = env_bool("MVR_ATTN_CHECKED", false);
  return v;
}

// Host copy of `count` int32 device values (none when ptr is null); false and
// an error message if the copy fails.
bool copy_table(const int32_t* dev, size_t count, hipStream_t stream, std::vector<int32_t>& host) {
  host.clear();
  if (!dev || count == 0) return true;
  host.resize(count);
  if (hipMemcpyAsync(host.data(), dev, count * sizeof(int32_t), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return true;
}

const int32_t* ptr_or_null(const std::vector<int32_t>& v) { return v.empty() ? nullptr : v.data(); }

struct TraceRange {
  bool on;
  explicit TraceRange(const char* name) : on(roctx_enabled()) {
    if (on) roctxRangePushA(name);
  }
  ~TraceRange() {
    if (on) roctxRangePop();
  }
};

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
  if (!mvr::head_dim_supported(a->head_dim))
    return fail(MVR_E_UNSUPPORTED, "head_dim %d is not supported (a multiple of 32 in [32, 256])", a->head_dim);
  if (a->page_size < 1) return fail(MVR_E_INVALID_ARGUMENT, "page_size must be positive");
  if (a->num_pages < 1) return fail(MVR_E_INVALID_ARGUMENT, "num_pages must be positive");
  if (a->max_q_len < 1) return fail(MVR_E_INVALID_ARGUMENT, "each forward input must contain at least one token");
  if (a->sum_seq_lens < 0 || (a->sum_seq_lens > 0 && a->sum_seq_lens > (int64_t)a->max_seq_len * a->num_seqs))
    return fail(MVR_E_INVALID_ARGUMENT, "sum_seq_lens %lld is outside [0, num_seqs * max_seq_len]",
                (long long)a->sum_seq_lens);
  if (a->max_seq_len < a->max_q_len)
    return fail(MVR_E_INVALID_ARGUMENT, "max_seq_len %d is smaller than max_q_len %d", a->max_seq_len, a->max_q_len);
  if (a->total_q < 0 || (a->total_q > 0 && (a->total_q < a->num_seqs ||
                                            a->total_q > (int64_t)a->num_seqs * a->max_q_len)))
    return fail(MVR_E_INVALID_ARGUMENT, "total_q %d is outside [num_seqs, num_seqs * max_q_len] (0: unknown)",
                a->total_q);
  if (a->num_seqs == 1 && !a->cu_q_lens && a->total_q > 0 && a->total_q < a->max_q_len)
    return fail(MVR_E_INVALID_ARGUMENT, "total_q %d is smaller than max_q_len %d, the q_len of a call without cu_q_lens",
                a->total_q, a->max_q_len);
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

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256; // no device to ask (sizing only): MI355X
  }
  return cus;
}

// What a launch's sequences hold, for sizing only: a class launch of a mixed
// batch spans every sequence of the call (its grid), but only the sequences of
// its class have rows there.  Defaults: every sequence, at the call's bounds.
struct LiveSeqs {
  int64_t count = 0;   // sequences with rows in this launch (0: num_seqs)
  int max_seq_len = 0; // their longest context (0: the call's max_seq_len)
  int64_t split_count = 0; // prefill kernel: sequences given key splits and partial slots (0: num_seqs)
};

mvr::PagedAttentionPlan make_plan(const mvr_paged_attention_args* a, bool allow_prefill = true,
                                  LiveSeqs live = LiveSeqs{}, bool force_prefill = false) {
  mvr::PagedAttentionPlan plan{};
  // Sizing inputs (the grid itself always covers num_seqs sequences and the
  // call's max_seq_len, which the kernels clamp device lengths to).
  const int64_t n_live = live.count > 0 && live.count < a->num_seqs ? live.count : a->num_seqs;
  const int len_live = live.max_seq_len > 0 && live.max_seq_len < a->max_seq_len ? live.max_seq_len : a->max_seq_len;
  plan.dtype = a->dtype;
  plan.head_dim = a->head_dim;
  const int group = a->num_q_heads / a->num_kv_heads;
  const int64_t rows_max = (int64_t)group * a->max_q_len;
  // Head dimensions other than 64 and 128: the split-context kernel in its
  // plain form (16-row tiles, 1-wavefront blocks, the merge pass) for
  // decode-sized calls; prefill-sized calls take the prefill kernel as at 64
  // and 128.
  const bool all_plans = mvr::head_dim_all_plans(a->head_dim);
  // Many query rows per KV head (chunked prefill): dense contraction, use the
  // LDS-shared 32x32 MFMA kernel (F16 32x32x16, F32 32x32x2).
  // MVR_ATTN_PREFILL_KERNEL=false keeps every call on the split-context kernel.
  static const bool prefill_enabled = env_bool("MVR_ATTN_PREFILL_KERNEL", true);
  // (Its loads take 16-token runs, 8 in F32, inside one page: page sizes
  // that are multiples of 16, as every size is after the repack; or, at
  // head_dim 64 and 128, each load's few whole token rows inside one page:
  // page sizes that prefill_token_pages_supported accepts.)
  const bool page_runs = a->page_size % mvr::kChunkTokens == 0;
  const bool prefill_pages =
      page_runs || mvr::prefill_token_pages_supported(a->page_size, a->num_kv_heads, a->head_dim,
                                                      a->dtype == MVR_DTYPE_F16 ? 2 : 4);
  // Other page sizes reach make_plan only for calls that the split-context
  // kernel serves, which then reads them in place (token pages), or that the
  // prefill kernel reads in place.
  plan.token_pages = !page_runs;
  if (allow_prefill && prefill_enabled && (rows_max > 64 || force_prefill) && prefill_pages &&
      mvr::prefill_head_dim_supported(a->head_dim)) {
    plan.prefill = true;
    plan.row_tiles = (int)((rows_max + mvr::kPrefillBlockRows - 1) / mvr::kPrefillBlockRows);
    const int64_t live_blocks = n_live * a->num_kv_heads * plan.row_tiles;
    const int key_tiles = (len_live + 31) / 32;
    static const int split_override = env_int("MVR_ATTN_PREFILL_SPLITS", 0);
    int64_t splits = split_override;
    if (splits <= 0) {
      // Split keys only while blocks leave CUs idle: one block per CU ran
      // faster than two half-length blocks plus the merge pass.
      splits = (int64_t)device_cus() / live_blocks;
      if (splits > key_tiles / 8) splits = key_tiles / 8; // keep >= 8 key tiles per split
    }
    if (splits > 8) splits = 8; // the merge holds one split per lane; 8 is plenty
    if (splits < 1) splits = 1;
    plan.kv_splits = (int)splits;
    // Wavefront groups per block.  Two groups share a block's 128 rows and
    // take alternating key tiles, two wavefronts per SIMD behind one barrier;
    // rows of more than 128 elements take one group (one wavefront per SIMD
    // holds their state).  F16 grids of at least 4 blocks per CU also take one
    // group, two independent blocks per CU.  Measured on fresh prompts (F16,
    // D=128), two groups -> one: Llama-3-8B 1 x 8192 589 -> 545 us, 4 x 2048
    // 188 -> 164, 1 x 4096 (1,024 blocks) 184-201 -> 172-184, Qwen2-7B 1 x
    // 8192 518 -> 497, 1 x 16384 1880 -> 1818; on smaller grids one group lost
    // up to 15% (the Qwen2-7B chunk, 224 blocks: 46.3 -> 53.0 us; Qwen2-7B 1 x
    // 4096, 896 blocks: 151-164 -> 171-178).  (One group in 32-token key tiles
    // instead of 64: 3-8% slower on these prompts.)
    // MVR_ATTN_PREFILL_GROUPS=1 or 2 forces a shape (2 only up to D=128).
    static const int groups_override = env_int("MVR_ATTN_PREFILL_GROUPS", 0);
    if (a->head_dim > 128)
      plan.prefill_groups = 1;
    else if (groups_override == 1 || groups_override == 2)
      plan.prefill_groups = groups_override;
    else
      plan.prefill_groups = a->dtype == MVR_DTYPE_F16 && live_blocks * splits >= 4LL * device_cus() ? 1 : 2;
    if (splits > 1) {
      const int64_t split_seqs = live.split_count > 0 && live.split_count < a->num_seqs ? live.split_count : a->num_seqs;
      const size_t prow = (size_t)(split_seqs * a->num_kv_heads * plan.row_tiles) * splits * mvr::kPrefillBlockRows;
      plan.partial_bytes = align_up(prow * a->head_dim * sizeof(float), 256) + align_up(prow * 2 * sizeof(float), 256);
    }
    return plan;
  }
  plan.row_blocks = rows_max <= 16 || !all_plans ? 1 : 2;
  const int tile_rows = 16 * plan.row_blocks;
  plan.row_tiles = (int)((rows_max + tile_rows - 1) / tile_rows);
  const int max_chunks = (a->max_seq_len + mvr::kChunkTokens - 1) / mvr::kChunkTokens; // the grid covers these
  const int live_chunks = (len_live + mvr::kChunkTokens - 1) / mvr::kChunkTokens;      // and sizes for these
  const int64_t base_units = (int64_t)a->num_seqs * a->num_kv_heads * plan.row_tiles;
  const bool ragged = a->sum_seq_lens > 0 && a->sum_seq_lens < (int64_t)len_live * n_live;
  int cpp = chunks_per_partition_override();
  const bool cpp_override_none = cpp <= 0;
  constexpr int kMaxPlannedParts = 128;
  // Kept for a dense ragged plan, which re-splits at a higher fill below.
  int64_t ragged_units_per_group = 0, ragged_total_chunks = 0, ragged_floor = 0;
  if (cpp <= 0) {
    // Split contexts so that the units fill the resident wavefront slots of
    // the device once: more partitions add merge traffic and a tail round,
    // fewer leave CUs idle.
    int64_t slots = target_waves_override();
    if (slots <= 0) {
      slots = mvr::paged_attention_resident_waves(plan.dtype, plan.head_dim, plan.row_blocks);
      if (slots <= 0) slots = 256 * 8; // no device to ask (sizing only)
      // F16 at head_dim 64 keeps 2 KiB per page and KV head, half the bytes
      // in flight per wavefront of head_dim 128, and its kernel fits four
      // wavefronts per SIMD: calls reading at least 256 MiB of K/V plan for
      // three per SIMD.  Measured (Qwen2-0.5B shape): uniform 64 x 16K (537
      // MB) 125.8 -> 109.5 us, 128 x U[1K,8K] (295 MB) 66.6 -> 62.0, 64 x
      // U[2K,16K] (295 MB) 65.6 -> 62.3; calls of 134 MB (64 x 4K, 16 x 16K)
      // lost 3%, F32 at head_dim 64 and head_dim 128 lost 1-10%.
      const int64_t tokens = a->sum_seq_lens > 0 ? a->sum_seq_lens : (int64_t)len_live * n_live;
      if (a->dtype == MVR_DTYPE_F16 && a->head_dim == 64 &&
          tokens * a->num_kv_heads * a->head_dim * 2 * 2 >= (int64_t)256 << 20)
        slots = slots * 3 / 2;
    }
    int64_t units_per_group = slots / ((int64_t)a->num_kv_heads * plan.row_tiles);
    if (units_per_group < 1) units_per_group = 1;
    int64_t c;
    if (ragged) {
      // Ragged lengths (known through sum_seq_lens): each sequence's last
      // partition is partial, and partition p of every sequence runs on the
      // same XCD, so the early partitions' XCDs carry more units than the
      // late ones'.  Plan for 80% of the slots to absorb both: on 16
      // sequences of 1K..16K tokens, 78% fill ran in 108 us and 95% in 132 us.
      const int64_t total_chunks =
          (a->sum_seq_lens + mvr::kChunkTokens - 1) / mvr::kChunkTokens + n_live / 2;
      int64_t u = units_per_group * 4 / 5;
      if (u < 1) u = 1;
      c = (total_chunks + u - 1) / u;
    } else {
      // Every sequence planned at max_seq_len: num_seqs * ceil(max_chunks / c) units.
      int64_t parts = units_per_group / n_live;
      if (parts < 1) parts = 1;
      c = (live_chunks + parts - 1) / parts;
    }
    // Floor: small batches are bound by each wavefront's serial chain of
    // chunk loads, so they split down to 4 chunks per wavefront (2 for
    // contexts up to 1024 tokens); measured 17.9 -> 12.1 us on one 512-token
    // F32 sequence and 24 -> 14 us on 8 sequences of 128..4096 tokens.
    const int64_t floor_cpp = live_chunks <= 64 ? 2 : 4;
    cpp = (int)(c < floor_cpp ? floor_cpp : (c > max_chunks ? max_chunks : c));
    if (ragged) {
      ragged_units_per_group = units_per_group;
      ragged_total_chunks = (a->sum_seq_lens + mvr::kChunkTokens - 1) / mvr::kChunkTokens + n_live / 2;
      ragged_floor = floor_cpp;
    }
  }
  if (cpp > max_chunks) cpp = max_chunks;
  plan.chunks_per_part = cpp;
  plan.max_parts = (max_chunks + cpp - 1) / cpp;
  // Block merge: a uniform batch split into at most one block's worth of
  // partitions (the batch-64 x 8K decode: 4 x 2048 tokens; one 512-token
  // sequence: 16 x 32 tokens) puts the partitions of one (sequence, KV head,
  // row tile) in one block of 4, 8 or 16 wavefronts and merges them in LDS,
  // without partials in HBM or a merge launch (about 8 us of launch gap and
  // kernel time).  Wavefronts past a tile's partitions idle through the
  // block's barriers, so a block is used only when at least three quarters of
  // its wavefronts hold a partition.  The wider blocks put a whole tile on
  // one CU, which suits F16 only: F32 products (v_mfma_f32_16x16x4_f32) made
  // one 512-token F32 sequence MFMA-bound on its CU, 14.8 us in 16-wavefront
  // blocks against 7.2 + 4.7 us for the same partitions spread over 8 CUs and
  // merged by a second launch.  Blocks of 16 wavefronts (128 VGPRs per lane)
  // for head_dim 64 only.  MVR_ATTN_BLOCK_MERGE=false keeps the separate merge.
  static const bool block_merge_enabled = env_bool("MVR_ATTN_BLOCK_MERGE", true);
  plan.block_waves = 0;
  // Token pages take blocks of 4 or 8 wavefronts, and none in F32 at D=128
  // (its registers would spill).
  const bool bm_shape = !plan.token_pages || a->dtype == MVR_DTYPE_F16 || a->head_dim != 128;
  if (block_merge_enabled && !ragged && plan.row_blocks == 1 && all_plans && bm_shape) {
    const int widest = a->dtype != MVR_DTYPE_F16 ? 4 : a->head_dim == 64 && !plan.token_pages ? 16 : 8;
    for (int w = 4; w <= widest && plan.block_waves == 0; w *= 2)
      if (plan.max_parts <= w && 4 * plan.max_parts >= 3 * w) plan.block_waves = w;
  }
  plan.block_merge = plan.block_waves > 0;
  // Dense layout for ragged batches with one row tile (dense_unit in
  // paged_attention.hip): the live units are numbered from 0, so in-order
  // dispatch balances them over the CUs and XCDs, where slot == partition
  // leaves a ragged batch's live early partitions piled onto some XCDs (64
  // sequences of 256..2048 tokens: 1.5x the mean load on two XCDs; rotating
  // each sequence's partitions instead left units starting up to 29 us late).
  // But slot == partition also keeps partition p of every sequence on one XCD,
  // so pages shared by several sequences (a common prefix) are read from HBM
  // once per XCD, and it suits few or long sequences: measured, the dense
  // layout took 64 ragged sequences from 79 to 72 us and the cascade suffix
  // pass of 64 sequences behind an 8K-token prompt from 119 to 110 us, but the
  // plain call on that shared prompt from 242 to 280 us, the 16-sequence
  // verify workload from 110 to 115 us (its cascade suffix pass from 127 to
  // 130) and 8 Qwen2-0.5B sequences from 14.2 to 15.0 us.  It is taken when
  // the batch has many sequences and most of the slot == partition grid
  // would hold no work (estimated from the length hint), which selects the
  // two winning cases and none of the others.  Token pages take it from 8
  // tokens per page (64 ragged sequences of 2,048..14,336 tokens in 8-token
  // pages 468 -> 431 us, the others within 1%); in 5-token pages it lost up
  // to 3.5% on shorter contexts.  MVR_ATTN_DENSE_RAGGED=false turns it off.
  static const bool dense_enabled = env_bool("MVR_ATTN_DENSE_RAGGED", true);
  bool dense = false;
  if (dense_enabled && ragged && plan.row_tiles == 1 && plan.max_parts > 1 && !plan.block_merge && n_live >= 32 &&
      (!plan.token_pages || a->page_size >= 8) && all_plans) {
    const int64_t chunk_tokens = (int64_t)mvr::kChunkTokens * plan.chunks_per_part;
    const int64_t est_live = (a->sum_seq_lens + chunk_tokens - 1) / chunk_tokens + n_live / 2;
    dense = est_live * 10 < (int64_t)a->num_seqs * plan.max_parts * 7; // live fraction < 0.7
  }
  plan.dense_parts = dense;
  if (dense && ragged_units_per_group > 0 && live_chunks > 64) {
    // Dense plans split for 120% of the resident slots instead of 80%:
    // in-order dispatch hands the extra units to whichever CU frees first,
    // and the layout has already given up the cross-sequence partition
    // alignment that more, shorter units would break.  Measured (F16 D=128
    // decode, U[L/8, L]): 128 x 8K 494 -> 440 us, 128 x 16K 1001 -> 901,
    // 32 x 4K 69 -> 65, 64 x 2K 73 -> 70; contexts up to 1K tokens (their
    // 2-chunk floor) lost 5% (256 x 512), so they keep 80%.  Key rows of more
    // than 256 bytes (F32 at head_dim 128: twice the bytes per unit of F16)
    // split for 180%: measured on F32 D=128, U[L/8, L] 32 x 4K 142 -> 136 us,
    // 48 x 8K 373 -> 340, 64 x 2K 150 -> 139, 64 x 8K 509 -> 460, 128 x 8K
    // 963 -> 937, 32 x 16K 500 -> 444; F16 and F32 D=64 lost 5-12% there.
    const bool wide_rows = (int64_t)a->head_dim * (a->dtype == MVR_DTYPE_F16 ? 2 : 4) > 256;
    int64_t u = ragged_units_per_group * (wide_rows ? 9 : 6) / 5;
    if (u < 1) u = 1;
    int64_t c = (ragged_total_chunks + u - 1) / u;
    if (c < ragged_floor) c = ragged_floor;
    if (c > max_chunks) c = max_chunks;
    plan.chunks_per_part = (int)c;
    plan.max_parts = (max_chunks + plan.chunks_per_part - 1) / plan.chunks_per_part;
  }
  // At most 128 partitions per tile: the merge kernel reads a row's partials
  // 32 per round trip, so a few long sequences over few KV heads split into
  // hundreds of partitions (one 32K-token sequence over 2 KV heads: 513) pay
  // more in the merge than the extra units save.  Measured (decode, one
  // query per sequence): Qwen2-0.5B F16 1 x 32K 29.1 -> 20.4 us, F32 31.6 ->
  // 29.5, 4 x 16K 23.4 -> 18.7; Llama-3-8B F16 1 x 32K 41.3 -> 34.6, F32
  // 65.5 -> 57.3; caps of 64 lost up to 30% on the Qwen2-0.5B ones.
  if (cpp_override_none && plan.max_parts > kMaxPlannedParts) {
    plan.chunks_per_part = (max_chunks + kMaxPlannedParts - 1) / kMaxPlannedParts;
    plan.max_parts = (max_chunks + plan.chunks_per_part - 1) / plan.chunks_per_part;
  }
  // Deep pipeline (three chunks in flight per wavefront) for the ragged plans
  // that keep slot == partition: their live wavefronts (planned at 80% of the
  // resident slots) do not fill the device and wait on load latency.  Measured
  // on F16 D=128 decode: ragged 8..16 sequences of up to 8K..32K tokens 14-19%
  // faster, 32 x 4K 5%, 24 x 12K and 16 x 32K unchanged; uniform batches gain
  // nothing, and short partitions (< 8 chunks: a 512-token F32 sequence, 8
  // Qwen2-0.5B sequences) lose 1-5% to the extra tail loads, so neither takes it.
  // MVR_ATTN_DEEP_PIPELINE=false turns it off.
  static const bool deep_enabled = env_bool("MVR_ATTN_DEEP_PIPELINE", true);
  const int elem_bytes = a->dtype == MVR_DTYPE_F16 ? 2 : 4;
  plan.deep_pipeline = deep_enabled && ragged && !dense && !plan.block_merge && !plan.token_pages && all_plans &&
                       plan.row_blocks == 1 && a->head_dim * elem_bytes <= 256 && plan.chunks_per_part >= 8;
  // No padding of max_parts.  Padding it to a multiple of 32 / gcd(Hkv * row
  // tiles, 32) made partition p of every sequence run on the same XCD (so
  // that pages shared by several sequences would meet in one L2), but the
  // padded partitions are empty and always land on the same XCDs: 128
  // sequences x 8K tokens (2 partitions padded to 4) left four XCDs idle,
  // 3,925 GB/s against 5,683 unpadded, and 48, 96 and 128 sequences gained
  // 34-52% at 512..8K tokens.  Unpadded was equal or better on every other
  // workload measured, the verify workload with its shared prefixes included.
  plan.num_units = base_units * (plan.block_merge ? plan.block_waves : plan.max_parts);
  // Block shape of plans without block merge: 4 wavefronts (4 KV heads of one
  // partition on one CU) or 1.  The dispatcher deals blocks to the 8 XCDs
  // round-robin, so with 4-wavefront blocks and a multiple of 32 units per
  // sequence, partition p of every sequence lands on the same two XCDs; in a
  // ragged batch the early partitions, live in every sequence, then pile onto
  // the same XCDs.  1-wavefront blocks with 8 KV heads put head h on XCD h:
  // every XCD gets the same work, and a page shared by several sequences is
  // read by one XCD per head slab.  Measured (HIP events, F16 D=128 unless
  // noted), 4 -> 1 wavefronts: 16 x U[1K,8K] 66.5 -> 56.7 us, F32 143.6 ->
  // 124.7, the 64-sequence shared-prompt batch 235.7 -> 224.4, dense plans
  // 1-6% faster; where the 4-wavefront layout already rotates over the XCDs
  // (16 x U[1K,16K], 8 x U[2K,32K], the verify batch) and on uniform batches
  // 1-wavefront blocks were 1-4% slower.  F32 units, twice the bytes of F16
  // ones, take 1-wavefront blocks whatever the layout (24 x U[1K,8K] D=128
  // 201 -> 171 us, 16 x U[2K,32K] 454 -> 408; one case of eight 3% slower).
  // Grids of fewer 4-wavefront blocks than CUs also take 1-wavefront blocks,
  // which spread them over more CUs (one 512-token F32 sequence 13.1 -> 12.1
  // us).  MVR_ATTN_UNIT_WAVES=1, 2 or 4 forces a shape.
  plan.unit_waves = 4;
  if (!plan.block_merge) {
    const int64_t units_per_seq = (int64_t)a->num_kv_heads * plan.row_tiles * plan.max_parts;
    if (plan.dense_parts || a->dtype != MVR_DTYPE_F16 || (ragged && units_per_seq % 32 == 0) ||
        plan.num_units < 4LL * device_cus())
      plan.unit_waves = 1;
    static const int unit_waves_override = env_int("MVR_ATTN_UNIT_WAVES", 0);
    if (unit_waves_override == 1 || unit_waves_override == 2 || unit_waves_override == 4)
      plan.unit_waves = unit_waves_override;
    if (plan.token_pages || !all_plans) plan.unit_waves = 1; // their one instantiation
  }
  plan.partial_bytes = 0;
  if (plan.max_parts > 1 && !plan.block_merge) {
    // [partial o][partial m, l]
    const size_t prow = (size_t)plan.num_units * tile_rows;
    plan.partial_bytes = align_up(prow * a->head_dim * sizeof(float), 256) + align_up(prow * 2 * sizeof(float), 256);
  }
  return plan;
}

} // namespace

namespace {

// The extra inputs of one launch: the passes of cascade attention, and the
// q_len class of one launch of a mixed batch (all null / 0 for a plain call).
struct LaunchExtras {
  int32_t class_q_min = 0, class_q_max = 0; // split-context kernel: sequences outside [min, max] (max 0: unbounded) are skipped
  // Prefill kernel: sequences in [skip_seq_lo, skip_seq_hi] with q_len <= skip_q_max (0: none) are skipped;
  // the main grid (key splits included) covers [seq_lo, seq_lo + seq_count) (count 0: all), and one
  // catch-up block per sequence of [catch_lo, catch_lo + catch_count) outside it computes that sequence unsplit.
  int32_t skip_seq_lo = 0, skip_seq_hi = -1, skip_q_max = 0;
  int32_t seq_lo = 0, seq_count = 0, catch_lo = 0, catch_count = 0;
  const int32_t* key_begin = nullptr; // suffix pass: first key of each sequence
  const int32_t* key_end = nullptr;   // prefix pass: keys [0, key_end) of each group
  float* state_o = nullptr;           // normalised fp32 rows instead of `out`
  float* state_lse = nullptr;
  int32_t state_tokens = 0;
  const float* prefix_o = nullptr;    // suffix pass: merge `out` rows with this prefix state
  const float* prefix_lse = nullptr;
  const int32_t* seq_prefix_len = nullptr;
};

// Launches the planned kernel(s); workspace ws holds plan.partial_bytes.
int launch_planned(const mvr_paged_attention_args* a, const mvr::PagedAttentionPlan& plan, void* ws,
                   const LaunchExtras& cp) {
  const float scale = a->scale > 0.f ? a->scale : (float)(1.0 / sqrt((double)a->head_dim));
  if (plan.prefill) {
    // The suffix pass is planned on the split-context kernel, which alone
    // merges rows with a prefix state.
    if (cp.prefix_o) return fail(MVR_E_INVALID_ARGUMENT, "internal: prefix merge planned on the prefill kernel");
    mvr::PrefillParams f{};
    f.q = a->q;
    f.q_stride_head = a->q_stride_head;
    f.q_stride_token = a->q_stride_token;
    f.key_pool = a->key_pool;
    f.value_pool = a->value_pool;
    f.block_tables = a->block_tables;
    f.block_table_stride = a->max_pages_per_seq;
    f.seq_lens = a->seq_lens;
    f.cu_q_lens = a->cu_q_lens;
    f.single_seq_len = a->max_seq_len;
    f.single_q_len = a->max_q_len;
    f.out = a->out;
    f.out_stride_head = a->out_stride_head;
    f.out_stride_token = a->out_stride_token;
    if (plan.partial_bytes) {
      const size_t prow = (size_t)(cp.seq_count ? cp.seq_count : a->num_seqs) * a->num_kv_heads *
                          plan.row_tiles * plan.kv_splits * mvr::kPrefillBlockRows;
      char* w = static_cast<char*>(ws);
      f.partial_o = reinterpret_cast<float*>(w);
      f.partial_ml = reinterpret_cast<float*>(w + align_up(prow * a->head_dim * sizeof(float), 256));
    }
    f.num_seqs = a->num_seqs;
    f.num_kv_heads = a->num_kv_heads;
    f.group_size = a->num_q_heads / a->num_kv_heads;
    f.page_size = a->page_size;
    mvr::page_divider(a->page_size, f.page_magic, f.page_magic_shift);
    f.row_tiles = plan.row_tiles;
    f.kv_splits = plan.kv_splits;
    f.groups = plan.prefill_groups;
    f.scale_log2 = scale * 1.4426950408889634f;
    f.key_end = cp.key_end;
    f.state_o = cp.state_o;
    f.state_lse = cp.state_lse;
    f.state_tokens = cp.state_tokens;
    if (cp.class_q_min > 0 || cp.class_q_max > 0)
      return fail(MVR_E_INVALID_ARGUMENT, "internal: q_len class filter planned on the prefill kernel");
    f.skip_seq_lo = cp.skip_seq_lo;
    f.skip_seq_hi = cp.skip_seq_hi;
    f.skip_q_max = cp.skip_q_max;
    f.seq_lo = cp.seq_lo;
    f.seq_count = cp.seq_count;
    f.catch_lo = cp.catch_lo;
    f.catch_count = cp.catch_count;
    TraceRange launch("attn-prefill-fused");
    hipError_t err = mvr::launch_paged_prefill(f, a->head_dim, a->dtype == MVR_DTYPE_F32, static_cast<hipStream_t>(a->stream));
    if (err != hipSuccess) return fail(MVR_E_HIP, "kernel launch failed: %s", hipGetErrorString(err));
    return MVR_OK;
  }

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
  mvr::page_divider(a->page_size, p.page_magic, p.page_magic_shift);
  p.out = a->out;
  p.out_stride_head = a->out_stride_head;
  p.out_stride_token = a->out_stride_token;
  if (plan.partial_bytes) {
    const size_t prow = (size_t)plan.num_units * 16 * plan.row_blocks;
    char* w = static_cast<char*>(ws);
    p.partial_o = reinterpret_cast<float*>(w);
    p.partial_ml = reinterpret_cast<float*>(w + align_up(prow * a->head_dim * sizeof(float), 256));
  }
  p.num_seqs = a->num_seqs;
  p.num_kv_heads = a->num_kv_heads;
  p.group_size = a->num_q_heads / a->num_kv_heads;
  p.page_size = a->page_size;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.key_begin = cp.key_begin;
  p.key_end = cp.key_end;
  p.state_o = cp.state_o;
  p.state_lse = cp.state_lse;
  p.state_tokens = cp.state_tokens;
  p.prefix_o = cp.prefix_o;
  p.prefix_lse = cp.prefix_lse;
  p.seq_prefix_len = cp.seq_prefix_len;
  p.class_q_min = cp.class_q_min;
  p.class_q_max = cp.class_q_max;

  TraceRange launch("attn-paged-fused"); // one launch replaces attn-qk / attn-mask-softmax / attn-paged-v
  hipError_t err = mvr::launch_paged_attention(plan, p, static_cast<hipStream_t>(a->stream));
  if (err != hipSuccess) return fail(MVR_E_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return MVR_OK;
}

int check_workspace(const mvr_paged_attention_args* a, size_t need) {
  if (a->workspace_bytes < need || (need && !a->workspace))
    return fail(MVR_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", a->workspace_bytes,
                need);
  if (need && ((uintptr_t)a->workspace & 255u)) return fail(MVR_E_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  return MVR_OK;
}

// One mvr_paged_attention call as one launch sequence, or two for a batch
// that may mix decode-sized requests (grouped rows G * q_len <= kSmallRows:
// one row tile of the split-context kernel) with prefill-sized ones.  Planned
// for its longest query, such a call would give every decode sequence the
// prefill kernel's 128-row tiles (or, in F32, 32-row split-context tiles with
// few context partitions).  Instead:
//   launch 0, the split-context kernel planned for the decode shape, over the
//     range of sequences [lo, hi] that holds the decode class (the whole call
//     without host tables), computing the sequences of that range whose device
//     q_len is at most its planned q_len (qmax);
//   launch 1, the prefill kernel planned for max_q_len, computing every
//     sequence that launch 0 does not (outside [lo, hi], or with q_len >
//     qmax): its main grid (key splits and partial slots included) covers the
//     range that holds the prefill class, and one catch-up block per
//     sequence covers the rest of [lo, hi] (each exits at once unless a stale
//     hint or a wrong guess put a prefill-sized request there, which it then
//     computes unsplit).
// Both launches decide from the device q_len, so each sequence is computed by
// exactly one of them whatever the host hints say: hints only shape the plans
// (with cu_q_lens_host a batch of one class runs as one unfiltered launch, and
// the class ranges and counts size each launch; seq_lens_host sizes the
// context splits), and a stale hint costs speed, never rows.
constexpr int kSmallRows = 32;

struct CallPlan {
  int n = 1;                       // launches (1 or 2)
  mvr_paged_attention_args part[2]; // each launch's view of the call
  mvr::PagedAttentionPlan plan[2];
  LaunchExtras extras[2];
  size_t offset[2] = {0, 0};       // workspace offset of each launch's partials
  size_t total = 0;
};

CallPlan make_call_plan(const mvr_paged_attention_args* a) {
  CallPlan c;
  c.part[0] = *a;
  c.plan[0] = make_plan(a);
  c.total = c.plan[0].partial_bytes;
  const int group = a->num_q_heads / a->num_kv_heads;
  const int small_q = kSmallRows / group; // largest q_len of the small class (0: no such class)
  if (a->num_seqs < 2 || small_q < 1 || a->max_q_len <= small_q) return c;
  if (!c.plan[0].prefill) return c; // launch 1 needs the prefill kernel
  const int32_t* cu = a->cu_q_lens_host;
  const int32_t* sl = a->seq_lens_host;
  int first[2] = {-1, -1}, last[2] = {-1, -1}, count[2] = {0, 0}, lmax[2] = {0, 0}, qmax = 0;
  int64_t lsum[2] = {0, 0};
  bool hinted = cu != nullptr;
  for (int s = 0; hinted && s < a->num_seqs; s++) {
    const int q = cu[s + 1] - cu[s];
    const int L = sl ? sl[s] : a->max_seq_len;
    // Hints that break the call's own bounds are ignored (the device tables
    // are what the kernels read; mvr_paged_attention_validate reports them).
    if (q < 1 || q > a->max_q_len || L < q || L > a->max_seq_len) {
      hinted = false;
      break;
    }
    const int k = q <= small_q ? 0 : 1;
    if (first[k] < 0) first[k] = s;
    last[k] = s;
    count[k]++;
    if (k == 0 && q > qmax) qmax = q;
    lsum[k] += L;
    if (L > lmax[k]) lmax[k] = L;
  }
  if (hinted && (count[0] == 0 || count[1] == 0)) return c; // one class: one unfiltered launch
  if (!hinted) {
    // Without hints the small class is the decode shape, up to 16 grouped
    // rows (one 16-row tile, the block-merge plans); longer queries,
    // speculative verification included, go to launch 1.  Launch 0 spans
    // every sequence.  The plans guess the rest from total_q: the tokens
    // beyond one per sequence are taken to fill prefill requests of
    // max_q_len each, packed after the decodes (the order in which
    // scheduler.rs:258-271 builds a batch).  A call whose tokens could fill
    // every sequence that way runs as one prefill launch (correct for any
    // mix, as is the guess: a prefill request outside the guessed tail is
    // computed unsplit by a catch-up block).
    qmax = 16 / group >= 1 ? 16 / group : small_q;
    // Unknown total_q: one prefill request.
    const int64_t excess = a->total_q > 0 ? (int64_t)a->total_q - a->num_seqs : 0;
    int64_t n_pref = excess > 0 ? (excess + a->max_q_len - 2) / (a->max_q_len - 1) : 1;
    if (n_pref >= a->num_seqs) return c;
    count[0] = a->num_seqs - (int)n_pref;
    count[1] = (int)n_pref;
    first[0] = 0;
    last[0] = a->num_seqs - 1;
    first[1] = a->num_seqs - (int)n_pref;
    last[1] = a->num_seqs - 1;
  }
  c.n = 2;
  // Launch 0: the decode range, its sequences at the call's bounds (the
  // kernels clamp a device seq_len to max_seq_len).
  mvr_paged_attention_args& p0 = c.part[0];
  p0 = *a;
  const int f = first[0];
  p0.num_seqs = last[0] - f + 1;
  // (null tables only when sizing a repacked call's workspace)
  p0.block_tables = a->block_tables ? a->block_tables + (int64_t)f * a->max_pages_per_seq : nullptr;
  p0.seq_lens = a->seq_lens ? a->seq_lens + f : nullptr;
  p0.cu_q_lens = a->cu_q_lens ? a->cu_q_lens + f : nullptr; // q_start stays the whole call's packed index
  p0.seq_lens_host = nullptr;
  p0.cu_q_lens_host = nullptr;
  p0.max_q_len = qmax;
  LiveSeqs live0;
  live0.count = count[0];
  if (hinted) {
    if (sl) live0.max_seq_len = lmax[0];
    p0.sum_seq_lens = sl ? lsum[0] : 0; // this class's keys (a speed hint)
  }
  c.plan[0] = make_plan(&p0, /*allow_prefill=*/false, live0);
  c.extras[0].class_q_min = 1;
  c.extras[0].class_q_max = qmax;
  // Launch 1: every sequence that launch 0 leaves.
  mvr_paged_attention_args& p1 = c.part[1];
  p1 = *a;
  p1.seq_lens_host = nullptr;
  p1.cu_q_lens_host = nullptr;
  LiveSeqs live1;
  live1.count = count[1];
  live1.split_count = last[1] - first[1] + 1;
  if (hinted) {
    if (sl) live1.max_seq_len = lmax[1];
    p1.sum_seq_lens = sl ? lsum[1] : 0;
  }
  c.plan[1] = make_plan(&p1, true, live1, /*force_prefill=*/true);
  LaunchExtras& e1 = c.extras[1];
  e1.skip_seq_lo = first[0];
  e1.skip_seq_hi = last[0];
  e1.skip_q_max = qmax;
  if (live1.split_count > 0 && live1.split_count < a->num_seqs) {
    // Main grid over the prefill range; the rest of the decode range gets a
    // catch-up block per sequence (it exits unless a stale hint put a
    // prefill-sized request there).
    e1.seq_lo = first[1];
    e1.seq_count = (int32_t)live1.split_count;
    e1.catch_lo = first[0];
    e1.catch_count = last[0] - first[0] + 1;
  }
  c.offset[0] = 0;
  c.offset[1] = align_up(c.plan[0].partial_bytes, 256);
  c.total = c.offset[1] + c.plan[1].partial_bytes;
  return c;
}

int launch_call(const CallPlan& c, char* ws) {
  for (int k = 0; k < c.n; k++) {
    const int rc = launch_planned(&c.part[k], c.plan[k], ws ? ws + c.offset[k] : nullptr, c.extras[k]);
    if (rc != MVR_OK) return rc;
  }
  return MVR_OK;
}

// Page sizes that are not a multiple of 16 (the reference allows any
// per_page_token_count; its own tests use 2 and 3) in a call that cannot read
// them in place (needs_repack): the call first repacks every sequence's
// tokens into 16-token pages in the workspace (launch_repack_pages: pages16
// pages per sequence at fixed stride, plus their block table), then runs the
// plan of that layout.  The attention is the same (only where the keys live
// changes), at the cost of one more copy of the K/V the batch reads.
// Workspace: [keys][values][block table][the plan's partials].
struct RepackPlan {
  mvr_paged_attention_args a16; // the call on the repacked layout (pointers into the workspace)
  CallPlan call;
  int pages16;
  size_t off_part, total;
};

// Page sizes that are not a multiple of 16 are read in place by the
// split-context kernel (token pages) down to 2 tokens per page, and by the
// chunked-prefill kernel where each of its loads' whole token rows lie in one
// page (prefill_token_pages_supported); a call that would use the
// chunked-prefill kernel with other page sizes, pages of one token, and pages
// of 2^31 elements or more over all KV heads (token pages keep offsets within
// a page in 32 bits) are repacked into 16-token pages first.
bool needs_repack(const mvr_paged_attention_args* a) {
  if (a->page_size % mvr::kChunkTokens == 0) return false;
  if (a->page_size < 2 || !mvr::head_dim_all_plans(a->head_dim) ||
      !mvr::token_page_offsets_fit(a->num_kv_heads, a->page_size, a->head_dim))
    return true;
  if (mvr::prefill_token_pages_supported(a->page_size, a->num_kv_heads, a->head_dim, a->dtype == MVR_DTYPE_F16 ? 2 : 4))
    return false;
  mvr_paged_attention_args b = *a;
  b.page_size = mvr::kChunkTokens; // the plan the repacked call would take
  const CallPlan c = make_call_plan(&b);
  for (int k = 0; k < c.n; k++)
    if (c.plan[k].prefill) return true;
  return false;
}

RepackPlan make_repack_plan(const mvr_paged_attention_args* a, char* ws) {
  RepackPlan r;
  r.pages16 = (a->max_seq_len + mvr::kChunkTokens - 1) / mvr::kChunkTokens;
  const int es = a->dtype == MVR_DTYPE_F16 ? 2 : 4;
  const size_t pool = (size_t)a->num_seqs * r.pages16 * a->num_kv_heads * mvr::kChunkTokens * a->head_dim * es;
  const size_t table = (size_t)a->num_seqs * r.pages16 * sizeof(int32_t);
  const size_t off_v = align_up(pool, 256), off_bt = off_v + align_up(pool, 256);
  r.off_part = off_bt + align_up(table, 256);
  r.a16 = *a;
  r.a16.page_size = mvr::kChunkTokens;
  r.a16.num_pages = (int64_t)a->num_seqs * r.pages16;
  r.a16.max_pages_per_seq = r.pages16;
  r.a16.key_pool = ws;
  r.a16.value_pool = ws ? ws + off_v : nullptr;
  r.a16.block_tables = ws ? reinterpret_cast<const int32_t*>(ws + off_bt) : nullptr;
  r.call = make_call_plan(&r.a16);
  r.total = r.off_part + r.call.total;
  return r;
}

// Cascade attention: a prefix pass over the groups' shared pages (each
// group's members' query rows as one virtual sequence whose keys end at the
// prefix) into a normalised fp32 state, then a suffix pass per sequence from
// its prefix on, whose final write merges each row with that state.
// Workspace: [prefix partials][suffix partials][prefix o][prefix lse].
struct CascadePlan {
  mvr_paged_attention_args pre, suf;
  mvr::PagedAttentionPlan pre_plan, suf_plan;
  int32_t state_tokens; // bound of the packed token count: state row stride
  size_t off_suf, off_a_o, off_a_lse, total;
};

int check_cascade(const mvr_paged_attention_args* a, const mvr_cascade_groups* g) {
  int rc = check_scalars(a);
  if (rc != MVR_OK) return rc;
  if (a->page_size % mvr::kChunkTokens != 0)
    return fail(MVR_E_UNSUPPORTED, "cascade attention needs a page_size that is a multiple of %d, not %d",
                mvr::kChunkTokens, a->page_size);
  if (!g) return fail(MVR_E_INVALID_ARGUMENT, "groups is null");
  if (g->num_groups < 0 || g->num_groups > a->num_seqs)
    return fail(MVR_E_INVALID_ARGUMENT, "num_groups %d is outside [0, num_seqs]", g->num_groups);
  if (!g->seq_prefix_lens) return fail(MVR_E_INVALID_ARGUMENT, "seq_prefix_lens is required");
  if (g->num_groups > 0) {
    if (!g->group_cu_q_lens || !g->group_prefix_lens || !g->group_block_tables)
      return fail(MVR_E_INVALID_ARGUMENT, "group tables are required when num_groups > 0");
    if (g->max_group_q_len < 1 || g->max_prefix_len < 0)
      return fail(MVR_E_INVALID_ARGUMENT, "max_group_q_len must be positive and max_prefix_len non-negative");
    if (g->max_prefix_len > a->max_seq_len)
      return fail(MVR_E_INVALID_ARGUMENT, "max_prefix_len %d exceeds max_seq_len %d", g->max_prefix_len, a->max_seq_len);
    if ((int64_t)g->max_group_q_len > (int64_t)a->num_seqs * a->max_q_len)
      return fail(MVR_E_INVALID_ARGUMENT, "max_group_q_len %d exceeds the packed token bound", g->max_group_q_len);
  }
  if (g->sum_prefix_lens < 0 || (a->sum_seq_lens > 0 && g->sum_prefix_lens > a->sum_seq_lens))
    return fail(MVR_E_INVALID_ARGUMENT, "sum_prefix_lens %lld is outside [0, sum_seq_lens]", (long long)g->sum_prefix_lens);
  return MVR_OK;
}

// Whether the cascade split is expected to beat the plain call.  The prefix
// pass reads each group's shared pages once instead of once per member, at
// a fixed cost: a second launch, per-row state written and read back, and a
// suffix pass whose partitions start at each sequence's prefix.  Measured
// (F16, Llama-3-8B shapes): 16 verify sequences of 1K..16K tokens in groups
// of 4 sharing 1K tokens (the shared reads are 9% of the plain call's key
// reads) took 124 us cascaded against 109 us plain; 64 sequences behind a
// shared 8K-token prompt (86%) ran 2.1x faster cascaded.  The call takes the
// plain path unless the saved reads are at least MVR_ATTN_CASCADE_MIN_SAVING
// percent (default 25; 0 always cascades) of the plain call's.  Saved reads
// are bounded below by sum_prefix_lens - num_groups * max_prefix_len, the
// plain call's reads above by sum_seq_lens (or num_seqs * max_seq_len);
// without the sum_prefix_lens hint the cascade runs as asked.
bool cascade_pays(const mvr_paged_attention_args* a, const mvr_cascade_groups* g) {
  static const int min_pct = env_int("MVR_ATTN_CASCADE_MIN_SAVING", 25);
  if (min_pct <= 0 || g->sum_prefix_lens <= 0) return true;
  const int64_t saved = g->sum_prefix_lens - (int64_t)g->num_groups * g->max_prefix_len;
  const int64_t reads = a->sum_seq_lens > 0 ? a->sum_seq_lens : (int64_t)a->num_seqs * a->max_seq_len;
  return saved > 0 && saved * 100 >= (int64_t)min_pct * reads;
}

CascadePlan make_cascade_plan(const mvr_paged_attention_args* a, const mvr_cascade_groups* g) {
  CascadePlan c;
  c.state_tokens = a->num_seqs * a->max_q_len;
  c.pre = *a;
  c.pre.num_seqs = g->num_groups > 0 ? g->num_groups : 1;
  c.pre.cu_q_lens = g->group_cu_q_lens;
  c.pre.seq_lens = nullptr; // the prefix pass derives each group's limits from its prefix length
  c.pre.block_tables = g->group_block_tables;
  c.pre.max_q_len = g->num_groups > 0 ? g->max_group_q_len : 1;
  c.pre.max_seq_len = (g->num_groups > 0 ? g->max_prefix_len : 1) + c.pre.max_q_len;
  c.pre.sum_seq_lens = 0;
  c.pre_plan = g->num_groups > 0 ? make_plan(&c.pre) : mvr::PagedAttentionPlan{};
  c.suf = *a;
  c.suf.sum_seq_lens =
      a->sum_seq_lens > 0 && g->sum_prefix_lens > 0 ? a->sum_seq_lens - g->sum_prefix_lens : a->sum_seq_lens;
  if (c.suf.sum_seq_lens >= (int64_t)a->max_seq_len * a->num_seqs) c.suf.sum_seq_lens = 0;
  // The suffix pass starts every sequence at its prefix: split-context kernel.
  c.suf_plan = make_plan(&c.suf, /*allow_prefill=*/false);
  const size_t so = (size_t)a->num_q_heads * c.state_tokens * a->head_dim * sizeof(float);
  const size_t sl = (size_t)a->num_q_heads * c.state_tokens * sizeof(float);
  c.off_suf = align_up(c.pre_plan.partial_bytes, 256);
  c.off_a_o = c.off_suf + align_up(c.suf_plan.partial_bytes, 256);
  c.off_a_lse = c.off_a_o + align_up(so, 256);
  c.total = c.off_a_lse + align_up(sl, 256);
  return c;
}

} // namespace

extern "C" {

int mvr_abi_version(void) { return MVR_ATTN_ABI_VERSION; }

const char* mvr_last_error(void) { return g_last_error; }

// ---------------------------------------------------------------------------
// RoPE + KV append
// ---------------------------------------------------------------------------

static int check_rope_append(const mvr_rope_append_args* a) {
  if (!a) return fail(MVR_E_INVALID_ARGUMENT, "args is null");
  if (a->dtype != MVR_DTYPE_F32 && a->dtype != MVR_DTYPE_F16)
    return fail(MVR_E_UNSUPPORTED, "dtype %d is not F32 (0) or F16 (1)", a->dtype);
  if (a->rope_type != MVR_ROPE_NEOX && a->rope_type != MVR_ROPE_INTERLEAVED)
    return fail(MVR_E_UNSUPPORTED, "rope_type %d is not Neox (0) or Interleaved (1)", a->rope_type);
  if (a->num_seqs < 1) return fail(MVR_E_INVALID_ARGUMENT, "forward requires at least one request");
  if (a->num_kv_heads < 1 || a->num_q_heads < 1 || a->num_q_heads % a->num_kv_heads != 0)
    return fail(MVR_E_INVALID_ARGUMENT, "num_q_heads %d is not a multiple of num_kv_heads %d", a->num_q_heads,
                a->num_kv_heads);
  if (a->head_dim < 8 || a->head_dim > 512 || a->head_dim % 8 != 0)
    return fail(MVR_E_UNSUPPORTED, "head_dim %d is not a multiple of 8 in [8, 512]", a->head_dim);
  if (a->page_size < 1) return fail(MVR_E_INVALID_ARGUMENT, "page_size must be positive");
  if (a->num_pages < 1) return fail(MVR_E_INVALID_ARGUMENT, "num_pages must be positive");
  if (a->total_q < 1) return fail(MVR_E_INVALID_ARGUMENT, "cannot append an empty KV-cache tensor"); // kv_cache/utils.rs:33-36
  if (a->num_seqs > a->total_q) return fail(MVR_E_INVALID_ARGUMENT, "cannot append an empty KV-cache tensor");
  if (a->max_seq_len < 1) return fail(MVR_E_INVALID_ARGUMENT, "max_seq_len must be positive");
  if (a->rope_len < a->max_seq_len)
    return fail(MVR_E_INVALID_ARGUMENT, "rotary tables hold %d positions, max_seq_len is %d", a->rope_len,
                a->max_seq_len);
  const int64_t pages_needed = (a->max_seq_len + (int64_t)a->page_size - 1) / a->page_size;
  if (a->max_pages_per_seq < pages_needed)
    return fail(MVR_E_PAGES_UNCOVERED, "block table rows of %d pages cannot hold %d tokens of %d-token pages",
                a->max_pages_per_seq, a->max_seq_len, a->page_size);
  if (a->num_seqs > 1 && (!a->seq_lens || !a->cu_q_lens))
    return fail(MVR_E_INVALID_ARGUMENT, "seq_lens and cu_q_lens are required when num_seqs > 1");
  if (!a->q || !a->k || !a->v || !a->cos_table || !a->sin_table || !a->block_tables || !a->q_out || !a->key_pool ||
      !a->value_pool)
    return fail(MVR_E_INVALID_ARGUMENT, "null tensor, table or pool pointer");
  const int64_t vec = 4; // every access moves 4 elements: 8 bytes (F16) or 16 bytes (F32)
  const size_t align = a->dtype == MVR_DTYPE_F16 ? 8 : 16;
  const void* ptrs[] = {a->q, a->k, a->v, a->cos_table, a->sin_table, a->q_out, a->key_pool, a->value_pool};
  for (const void* ptr : ptrs)
    if ((uintptr_t)ptr % align)
      return fail(MVR_E_INVALID_ARGUMENT, "tensors, tables and pools must be %zu-byte aligned", align);
  const int64_t strides[] = {a->q_stride_head, a->q_stride_token, a->k_stride_head,     a->k_stride_token,
                             a->v_stride_head, a->v_stride_token, a->q_out_stride_head, a->q_out_stride_token};
  for (int64_t st : strides)
    if (st % vec) return fail(MVR_E_INVALID_ARGUMENT, "strides must be multiples of %lld elements", (long long)vec);
  return MVR_OK;
}

int mvr_rope_append(const mvr_rope_append_args* a) {
  // The reference traces forward_rope of the query and the key (trace.rs:77-79,
  // common.rs:306-307, 351) and then the cache append (trace.rs:81-83,
  // common.rs:310); here one launch does all three, so the append range
  // (around the launch) sits inside the rope range.
  TraceRange range("attn-rope tensor=query,key");
  g_last_error[0] = 0;
  int rc = check_rope_append(a);
  if (rc != MVR_OK) return rc;
  if (checked_mode()) {
    hipStream_t st = static_cast<hipStream_t>(a->stream);
    std::vector<int32_t> bt, sl, cu;
    if (!copy_table(a->block_tables, (size_t)a->num_seqs * a->max_pages_per_seq, st, bt) ||
        !copy_table(a->seq_lens, (size_t)a->num_seqs, st, sl) || !copy_table(a->cu_q_lens, (size_t)a->num_seqs + 1, st, cu))
      return fail(MVR_E_HIP, "checked mode: copying the device tables to the host failed");
    rc = mvr_rope_append_validate(a, ptr_or_null(bt), ptr_or_null(sl), ptr_or_null(cu), nullptr);
    if (rc != MVR_OK) return rc;
  }
  TraceRange append("attn-cache operation=append");
  mvr::RopeAppendParams p{};
  p.q = a->q;
  p.q_stride_head = a->q_stride_head;
  p.q_stride_token = a->q_stride_token;
  p.k = a->k;
  p.k_stride_head = a->k_stride_head;
  p.k_stride_token = a->k_stride_token;
  p.v = a->v;
  p.v_stride_head = a->v_stride_head;
  p.v_stride_token = a->v_stride_token;
  p.cos_table = a->cos_table;
  p.sin_table = a->sin_table;
  p.block_tables = a->block_tables;
  p.block_table_stride = a->max_pages_per_seq;
  p.seq_lens = a->seq_lens;
  p.cu_q_lens = a->cu_q_lens;
  p.single_seq_len = a->max_seq_len;
  p.q_out = a->q_out;
  p.q_out_stride_head = a->q_out_stride_head;
  p.q_out_stride_token = a->q_out_stride_token;
  p.key_pool = a->key_pool;
  p.value_pool = a->value_pool;
  p.num_seqs = a->num_seqs;
  p.num_q_heads = a->num_q_heads;
  p.num_kv_heads = a->num_kv_heads;
  p.head_dim = a->head_dim;
  p.page_size = a->page_size;
  p.total_q = a->total_q;
  hipError_t err = mvr::launch_rope_append(p, a->dtype, a->rope_type, static_cast<hipStream_t>(a->stream));
  if (err != hipSuccess) return fail(MVR_E_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return MVR_OK;
}

int mvr_rope_append_validate(const mvr_rope_append_args* a, const int32_t* block_tables_host,
                             const int32_t* seq_lens_host, const int32_t* cu_q_lens_host,
                             const uint8_t* page_writable_host) {
  g_last_error[0] = 0;
  int rc = check_rope_append(a);
  if (rc != MVR_OK) return rc;
  if (cu_q_lens_host) {
    if (cu_q_lens_host[0] != 0) return fail(MVR_E_INVALID_ARGUMENT, "cu_q_lens[0] must be 0");
    if (cu_q_lens_host[a->num_seqs] != a->total_q)
      return fail(MVR_E_INVALID_ARGUMENT, "cu_q_lens[num_seqs] = %d, total_q = %d", cu_q_lens_host[a->num_seqs],
                  a->total_q);
  }
  // Pages written by an earlier request of this call (a page is PendingWrite
  // for one request only; two writers would race).
  uint8_t* owner_seen = nullptr;
  if (block_tables_host) {
    owner_seen = static_cast<uint8_t*>(calloc((size_t)a->num_pages, 1));
    if (!owner_seen) return fail(MVR_E_INVALID_ARGUMENT, "out of host memory");
  }
  rc = MVR_OK;
  for (int s = 0; s < a->num_seqs && rc == MVR_OK; s++) {
    const int q_len = cu_q_lens_host ? cu_q_lens_host[s + 1] - cu_q_lens_host[s] : (a->num_seqs == 1 ? a->total_q : -1);
    const int seq_len = seq_lens_host ? seq_lens_host[s] : (a->num_seqs == 1 ? a->max_seq_len : -1);
    if (q_len == 0 || (q_len < 0 && cu_q_lens_host)) {
      rc = fail(MVR_E_INVALID_ARGUMENT, "cannot append an empty KV-cache tensor"); // kv_cache/utils.rs:33-36
      break;
    }
    if (seq_len < 0 || q_len < 0) continue;
    if (seq_len > a->max_seq_len) {
      rc = fail(MVR_E_INVALID_ARGUMENT, "request %d has seq_len %d > max_seq_len %d", s, seq_len, a->max_seq_len);
      break;
    }
    if (seq_len < q_len) {
      rc = fail(MVR_E_LENGTH_MISMATCH, "KV-cache contains %d tokens after appending %d", seq_len, q_len);
      break;
    }
    if (!block_tables_host) continue;
    const int first = (seq_len - q_len) / a->page_size, last = (seq_len - 1) / a->page_size;
    for (int pi = first; pi <= last; pi++) {
      const int32_t id = block_tables_host[(int64_t)s * a->max_pages_per_seq + pi];
      if (id < 0 || id >= a->num_pages) {
        rc = fail(MVR_E_PAGE_ID, "request %d page %d has id %d outside a pool of %lld pages", s, pi, id,
                  (long long)a->num_pages);
        break;
      }
      if (page_writable_host && !page_writable_host[id]) {
        rc = fail(MVR_E_READ_ONLY_PAGE, "cannot mutate written physical page %d", id); // physical_page_pool.rs:197-201
        break;
      }
      if (owner_seen[id]) {
        rc = fail(MVR_E_INVALID_ARGUMENT, "page %d is written by more than one request", id);
        break;
      }
      owner_seen[id] = 1;
    }
  }
  free(owner_seen);
  return rc;
}

size_t mvr_paged_attention_workspace_size(const mvr_paged_attention_args* args) {
  if (check_scalars(args) != MVR_OK) return 0;
  if (needs_repack(args)) return make_repack_plan(args, nullptr).total;
  return make_call_plan(args).total;
}

// MVR_ATTN_CHECKED: the device tables of an attention call through
// mvr_paged_attention_validate.
static int checked_attention_tables(const mvr_paged_attention_args* a) {
  hipStream_t st = static_cast<hipStream_t>(a->stream);
  std::vector<int32_t> bt, sl, cu;
  if (!copy_table(a->block_tables, (size_t)a->num_seqs * a->max_pages_per_seq, st, bt) ||
      !copy_table(a->seq_lens, (size_t)a->num_seqs, st, sl) ||
      !copy_table(a->cu_q_lens, (size_t)a->num_seqs + 1, st, cu))
    return fail(MVR_E_HIP, "checked mode: copying the device tables to the host failed");
  // The host hints must hold the device tables' values (they shape the plan).
  if (a->seq_lens_host && !sl.empty())
    for (int s = 0; s < a->num_seqs; s++)
      if (a->seq_lens_host[s] != sl[s])
        return fail(MVR_E_INVALID_ARGUMENT, "seq_lens_host[%d] = %d differs from the device seq_lens (%d)", s,
                    a->seq_lens_host[s], sl[s]);
  if (a->cu_q_lens_host && !cu.empty())
    for (int s = 0; s <= a->num_seqs; s++)
      if (a->cu_q_lens_host[s] != cu[s])
        return fail(MVR_E_INVALID_ARGUMENT, "cu_q_lens_host[%d] = %d differs from the device cu_q_lens (%d)", s,
                    a->cu_q_lens_host[s], cu[s]);
  if (a->total_q > 0 && !cu.empty() && cu[a->num_seqs] > a->total_q)
    return fail(MVR_E_INVALID_ARGUMENT, "the device cu_q_lens[num_seqs] = %d exceeds total_q = %d", cu[a->num_seqs],
                a->total_q);
  return mvr_paged_attention_validate(a, ptr_or_null(bt), ptr_or_null(sl), ptr_or_null(cu));
}

// Device address of `scratch` on the current device: looked up with that
// device current on its first call there, then kept per device (each device
// holds its own copy at its own address).  Null (error set) if the lookup
// fails.
static void* noalloc_scratch() {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> addr[kMaxDevices];
  static std::mutex lookup;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    fail(MVR_E_HIP, "no current device (or device index >= %d) for the static scratch", kMaxDevices);
    return nullptr;
  }
  void* p = addr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> guard(lookup);
  p = addr[dev].load(std::memory_order_relaxed);
  if (!p) {
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p) {
      (void)hipGetLastError();
      fail(MVR_E_HIP, "hipGetSymbolAddress of the static scratch failed on device %d: %s", dev, hipGetErrorString(err));
      return nullptr;
    }
    addr[dev].store(p, std::memory_order_release);
  }
  return p;
}

// The launches of one mvr_paged_attention call on the workspace the
// arguments carry (scalar checks already done).
static int paged_attention_launches(const mvr_paged_attention_args* a) {
  int rc;
  if (needs_repack(a)) {
    const RepackPlan r = make_repack_plan(a, static_cast<char*>(a->workspace));
    rc = check_workspace(a, r.total);
    if (rc != MVR_OK) return rc;
    const int es = a->dtype == MVR_DTYPE_F16 ? 2 : 4;
    TraceRange repack("attn-cache operation=access result_layout=repacked");
    hipError_t err = mvr::launch_repack_pages(
        a->key_pool, a->value_pool, a->block_tables, a->max_pages_per_seq, a->seq_lens, a->max_seq_len, a->num_seqs,
        a->num_kv_heads, a->page_size, a->head_dim, es, r.pages16, const_cast<void*>(r.a16.key_pool),
        const_cast<void*>(r.a16.value_pool), const_cast<int32_t*>(r.a16.block_tables), static_cast<hipStream_t>(a->stream));
    if (err != hipSuccess) return fail(MVR_E_HIP, "kernel launch failed: %s", hipGetErrorString(err));
    return launch_call(r.call, static_cast<char*>(a->workspace) + r.off_part);
  }
  const CallPlan c = make_call_plan(a);
  rc = check_workspace(a, c.total);
  if (rc != MVR_OK) return rc;
  return launch_call(c, static_cast<char*>(a->workspace));
}

int mvr_paged_attention(const mvr_paged_attention_args* a) {
  TraceRange range("attn"); // trace.rs:64
  g_last_error[0] = 0;
  int rc = check_scalars(a);
  if (rc != MVR_OK) return rc;
  if (checked_mode() && (rc = checked_attention_tables(a)) != MVR_OK) return rc;
  return paged_attention_launches(a);
}

int mvr_paged_attention_noalloc(const mvr_paged_attention_args* a) {
  TraceRange range("attn"); // trace.rs:64
  g_last_error[0] = 0;
  int rc = check_scalars(a);
  if (rc != MVR_OK) return rc;
  const size_t need =
      needs_repack(a) ? make_repack_plan(a, nullptr).total : make_call_plan(a).total;
  if (need > (size_t)MVR_NOALLOC_SCRATCH_BYTES)
    return fail(MVR_E_WORKSPACE,
                "this call needs %zu bytes of scratch, more than the %zu bytes of the library's static scratch; "
                "call mvr_paged_attention with a workspace instead",
                need, (size_t)MVR_NOALLOC_SCRATCH_BYTES);
  mvr_paged_attention_args b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  if (need) {
    b.workspace = noalloc_scratch();
    if (!b.workspace) return MVR_E_HIP;
    b.workspace_bytes = MVR_NOALLOC_SCRATCH_BYTES;
  }
  return paged_attention_launches(&b);
}

size_t mvr_paged_attention_cascade_workspace_size(const mvr_paged_attention_args* args,
                                                  const mvr_cascade_groups* groups) {
  if (check_cascade(args, groups) != MVR_OK) return 0;
  if (!cascade_pays(args, groups)) return mvr_paged_attention_workspace_size(args);
  return make_cascade_plan(args, groups).total;
}

int mvr_paged_attention_cascade(const mvr_paged_attention_args* a, const mvr_cascade_groups* g) {
  TraceRange range("attn");
  g_last_error[0] = 0;
  int rc = check_cascade(a, g);
  if (rc != MVR_OK) return rc;
  if (checked_mode()) {
    hipStream_t st = static_cast<hipStream_t>(a->stream);
    const size_t ng = g->num_groups > 0 ? (size_t)g->num_groups : 0;
    std::vector<int32_t> bt, sl, cu, gcu, gpre, gbt, spre;
    if (!copy_table(a->block_tables, (size_t)a->num_seqs * a->max_pages_per_seq, st, bt) ||
        !copy_table(a->seq_lens, (size_t)a->num_seqs, st, sl) || !copy_table(a->cu_q_lens, (size_t)a->num_seqs + 1, st, cu) ||
        !copy_table(ng ? g->group_cu_q_lens : nullptr, ng + 1, st, gcu) ||
        !copy_table(ng ? g->group_prefix_lens : nullptr, ng, st, gpre) ||
        !copy_table(ng ? g->group_block_tables : nullptr, ng * a->max_pages_per_seq, st, gbt) ||
        !copy_table(g->seq_prefix_lens, (size_t)a->num_seqs, st, spre))
      return fail(MVR_E_HIP, "checked mode: copying the device tables to the host failed");
    rc = mvr_paged_attention_cascade_validate(a, g, ptr_or_null(bt), ptr_or_null(sl), ptr_or_null(cu),
                                              ptr_or_null(gcu), ptr_or_null(gpre), ptr_or_null(gbt),
                                              ptr_or_null(spre));
    if (rc != MVR_OK) return rc;
  }
  if (!cascade_pays(a, g)) return paged_attention_launches(a);
  const CascadePlan c = make_cascade_plan(a, g);
  rc = check_workspace(a, c.total);
  if (rc != MVR_OK) return rc;
  char* ws = static_cast<char*>(a->workspace);
  float* a_o = reinterpret_cast<float*>(ws + c.off_a_o);
  float* a_lse = reinterpret_cast<float*>(ws + c.off_a_lse);
  if (g->num_groups > 0) {
    LaunchExtras pre;
    pre.key_end = g->group_prefix_lens;
    pre.state_o = a_o;
    pre.state_lse = a_lse;
    pre.state_tokens = c.state_tokens;
    rc = launch_planned(&c.pre, c.pre_plan, ws, pre);
    if (rc != MVR_OK) return rc;
  }
  // The suffix pass writes `out`, each row merged with its prefix state.
  LaunchExtras suf;
  suf.key_begin = g->seq_prefix_lens;
  suf.state_tokens = c.state_tokens;
  if (g->num_groups > 0) {
    suf.prefix_o = a_o;
    suf.prefix_lse = a_lse;
    suf.seq_prefix_len = g->seq_prefix_lens;
  }
  return launch_planned(&c.suf, c.suf_plan, ws + c.off_suf, suf);
}

int mvr_paged_attention_cascade_validate(const mvr_paged_attention_args* a, const mvr_cascade_groups* g,
                                         const int32_t* bt, const int32_t* seq_lens, const int32_t* cu,
                                         const int32_t* gcu, const int32_t* gpre, const int32_t* gbt,
                                         const int32_t* spre) {
  g_last_error[0] = 0;
  int rc = check_cascade(a, g);
  if (rc != MVR_OK) return rc;
  rc = mvr_paged_attention_validate(a, bt, seq_lens, cu);
  if (rc != MVR_OK) return rc;
  if (!gcu || !cu) return MVR_OK;
  const int ng = g->num_groups;
  int s = 0; // sequences before the current group must carry no prefix
  for (int gi = 0; gi < ng; gi++) {
    if (gcu[gi + 1] <= gcu[gi])
      return fail(MVR_E_INVALID_ARGUMENT, "group %d has no query tokens", gi);
    if (gcu[gi + 1] - gcu[gi] > g->max_group_q_len)
      return fail(MVR_E_INVALID_ARGUMENT, "group %d has %d query tokens > max_group_q_len %d", gi,
                  gcu[gi + 1] - gcu[gi], g->max_group_q_len);
    // Members: the consecutive sequences whose tokens span [gcu[gi], gcu[gi+1]).
    while (s < a->num_seqs && cu[s] < gcu[gi]) {
      if (spre && spre[s] != 0)
        return fail(MVR_E_INVALID_ARGUMENT, "sequence %d is in no group but has seq_prefix_lens %d", s, spre[s]);
      s++;
    }
    if (s >= a->num_seqs || cu[s] != gcu[gi])
      return fail(MVR_E_INVALID_ARGUMENT, "group %d does not start at a sequence boundary", gi);
    const int pre = gpre ? gpre[gi] : -1;
    if (gpre && (pre < 0 || pre % a->page_size || pre > g->max_prefix_len))
      return fail(MVR_E_INVALID_ARGUMENT, "group %d prefix %d is not a multiple of page_size %d within max_prefix_len",
                  gi, pre, a->page_size);
    for (; s < a->num_seqs && cu[s] < gcu[gi + 1]; s++) {
      if (cu[s + 1] > gcu[gi + 1])
        return fail(MVR_E_INVALID_ARGUMENT, "group %d does not end at a sequence boundary", gi);
      if (spre && gpre && spre[s] != pre)
        return fail(MVR_E_INVALID_ARGUMENT, "sequence %d has seq_prefix_lens %d, its group's prefix is %d", s, spre[s], pre);
      if (gpre && seq_lens) {
        const int cached = seq_lens[s] - (cu[s + 1] - cu[s]);
        if (pre > cached)
          return fail(MVR_E_INVALID_ARGUMENT, "group %d prefix %d exceeds sequence %d's %d cached tokens", gi, pre, s, cached);
      }
      if (gpre && bt && gbt)
        for (int pi = 0; pi < pre / a->page_size; pi++)
          if (bt[(int64_t)s * a->max_pages_per_seq + pi] != gbt[(int64_t)gi * a->max_pages_per_seq + pi])
            return fail(MVR_E_INVALID_ARGUMENT, "sequence %d page %d differs from its group's shared page", s, pi);
    }
  }
  for (; s < a->num_seqs; s++)
    if (spre && spre[s] != 0)
      return fail(MVR_E_INVALID_ARGUMENT, "sequence %d is in no group but has seq_prefix_lens %d", s, spre[s]);
  return MVR_OK;
}

int mvr_paged_attention_validate(const mvr_paged_attention_args* a, const int32_t* block_tables_host,
                                 const int32_t* seq_lens_host, const int32_t* cu_q_lens_host) {
  g_last_error[0] = 0;
  int rc = check_scalars(a);
  if (rc != MVR_OK) return rc;
  if (cu_q_lens_host && a->total_q > 0 && cu_q_lens_host[a->num_seqs] > a->total_q)
    return fail(MVR_E_INVALID_ARGUMENT, "cu_q_lens[num_seqs] = %d exceeds total_q = %d", cu_q_lens_host[a->num_seqs],
                a->total_q);
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
  a->total_q = dims->q_len;
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

int mvr_reconstruct_contiguous(int32_t dtype, const void* pool, int64_t page_count, int32_t num_kv_heads,
                               int32_t per_page_token_count, int32_t head_dim, const int32_t* page_ids,
                               int32_t num_page_ids, int32_t cached_token_count, void* out, void* stream) {
  // trace.rs:85-92: the access that materialises contiguous K/V (common.rs:386)
  TraceRange range("attn-cache operation=access result_layout=contiguous");
  g_last_error[0] = 0;
  if (dtype != MVR_DTYPE_F32 && dtype != MVR_DTYPE_F16)
    return fail(MVR_E_UNSUPPORTED, "dtype %d is not F32 (0) or F16 (1)", dtype);
  if (cached_token_count <= 0 || num_page_ids <= 0)
    return fail(MVR_E_INVALID_ARGUMENT, "cannot reconstruct an empty KV cache"); // paged_cache.rs:383-385
  if (num_kv_heads < 1 || per_page_token_count < 1 || head_dim < 1 || page_count < 1)
    return fail(MVR_E_INVALID_ARGUMENT, "invalid pool geometry");
  const int64_t covered = (int64_t)num_page_ids * per_page_token_count;
  if (covered < cached_token_count)
    return fail(MVR_E_PAGES_UNCOVERED,
                "paged KV cache contains fewer pages than its sequence length, leaving %lld tokens uncovered",
                (long long)(cached_token_count - covered));
  if (!pool || !page_ids || !out) return fail(MVR_E_INVALID_ARGUMENT, "null pool, page ids or output pointer");
  const int es = dtype == MVR_DTYPE_F16 ? 2 : 4;
  hipError_t err = mvr::launch_gather_pages(pool, page_ids, num_kv_heads, per_page_token_count, head_dim, es,
                                            cached_token_count, out, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(MVR_E_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return MVR_OK;
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
