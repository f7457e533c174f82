/*
 * mvr_attn — MI355X (gfx950) page-wise attention over a paged KV cache.
 *
 * C ABI for mini-vllm-rs's attention hot path.  It replaces
 *   - the CPU-only page-wise attention, forward_paged_attention
 *     (src/models/backends/common.rs:739-817, reached through
 *     forward_cpu_paged_attention, common.rs:426-464), and
 *   - the GPU gather-to-contiguous fallback, reconstruct_contiguous_tensor
 *     (src/model_runner/server/kv_cache/paged_cache.rs:363-391) followed by
 *     forward_contiguous_attention (common.rs:703-737).
 *
 * Data contract (src/models/mod.rs:56-100, kv_cache/utils.rs:55-74):
 *   key_pool / value_pool: [num_pages, 1, num_kv_heads, page_size, head_dim],
 *     contiguous, in the activation dtype (F32 or F16).
 *   block_tables: int32 [num_seqs, max_pages_per_seq]; row s holds the
 *     request's page_ids in logical order (PagedCacheLayout::page_ids).
 *   seq_lens: int32 [num_seqs] = cached_token_count, which already includes
 *     the request's current query tokens (common.rs:447-454).
 *   cu_q_lens: int32 [num_seqs + 1], prefix sums of q_len
 *     (ForwardContext::q_start_index, common.rs:603-626).
 *   q / out: element (q head h, packed token n, dim d) at
 *     h*stride_head + n*stride_token + d.  The reference's packed layout
 *     [1, Hq, packed_q_len, D] has stride_head = packed_q_len*D,
 *     stride_token = D (common.rs:268-275, 326-332).
 *   Q head h reads KV head h / (num_q_heads / num_kv_heads)
 *     (common.rs:819-859).
 *   Query i of a request (0-based within the request) sees keys
 *     0 ..= seq_len - q_len + i (common.rs:948-965).
 *
 * Every call is stream-ordered and asynchronous and allocates nothing.  Its
 * only global state is a thread-local error string, environment flags read
 * once, and a per-device cache of the runtime's occupancy answer (atomics,
 * each written with a value that never changes), so several threads may
 * drive several devices concurrently.  Functions return MVR_OK (0) or a
 * negative MVR_E_* code; mvr_last_error() describes the last failure on the
 * calling thread.
 *
 * Device tables (block tables, lengths, group tables) are trusted by the
 * launching entry points; the *_validate functions check host copies.  With
 * MVR_ATTN_CHECKED=true in the environment (a development mode) every
 * launching call first copies its device tables back, waits for its stream
 * and runs those checks, returning their error instead of launching.  The
 * kernels clamp a device seq_len above max_seq_len to max_seq_len, so such a
 * table reads no page outside its block-table row.
 */
#ifndef MVR_ATTN_H
#define MVR_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVR_ATTN_ABI_VERSION 3

/* ActivationDType (src/model_runner/mod.rs:331-351): F32 or F16 only. */
typedef enum { MVR_DTYPE_F32 = 0, MVR_DTYPE_F16 = 1 } mvr_dtype;

typedef enum {
  MVR_OK = 0,
  MVR_E_INVALID_ARGUMENT = -1,
  MVR_E_UNSUPPORTED = -2,
  /* common.rs:447-454: "paged KV cache reports sequence length X, expected Y" */
  MVR_E_LENGTH_MISMATCH = -3,
  /* common.rs:776-781: "paged KV cache contains fewer pages than its sequence
     length, leaving N tokens uncovered" */
  MVR_E_PAGES_UNCOVERED = -4,
  /* a page id outside [0, num_pages) (Tensor::narrow fails in the reference) */
  MVR_E_PAGE_ID = -5,
  MVR_E_WORKSPACE = -6,
  MVR_E_HIP = -7,
  /* physical_page_pool.rs:197-201: "cannot mutate written physical page N" */
  MVR_E_READ_ONLY_PAGE = -8
} mvr_status;

typedef struct mvr_paged_attention_args {
  int32_t dtype;             /* mvr_dtype */
  int32_t num_seqs;          /* requests packed in this call, >= 1 */
  int32_t num_q_heads;
  int32_t num_kv_heads;      /* divides num_q_heads */
  int32_t head_dim;          /* a multiple of 32 in [32, 256]; 64 and 128 take every plan, the others the
                                split-context kernel with its merge pass and the chunked-prefill kernel */
  int32_t page_size;         /* per_page_token_count, any positive value; sizes that are not a multiple of
                                16 are read in place by decode-sized calls (2 tokens or more) and, at
                                head_dim 64 and 128, by prefill-sized calls whose page size is a multiple
                                of the tokens one prefill load covers (F16: 4 at D=128, 8 at D=64; F32: 2
                                at D=128, 4 at D=64); the others, and 1-token pages, are repacked into
                                16-token pages in the workspace first */
  int64_t num_pages;         /* page_count of each pool */
  int32_t max_pages_per_seq; /* row stride of block_tables */
  int32_t max_q_len;         /* >= every q_len (host-side bound, sizes the grid) */
  int32_t max_seq_len;       /* >= every seq_len (host-side bound, sizes the grid) */
  float scale;               /* softmax scale; 0 selects 1/sqrt(head_dim) as the reference does */
  const void* q;
  int64_t q_stride_head;     /* elements */
  int64_t q_stride_token;    /* elements */
  const void* key_pool;
  const void* value_pool;
  const int32_t* block_tables; /* device */
  const int32_t* seq_lens;     /* device; NULL allowed when num_seqs == 1: seq_len = max_seq_len */
  const int32_t* cu_q_lens;    /* device; NULL allowed when num_seqs == 1: q_len = max_q_len */
  void* out;
  int64_t out_stride_head;   /* elements */
  int64_t out_stride_token;  /* elements */
  void* workspace;           /* device scratch for split-context partials */
  size_t workspace_bytes;
  void* stream;              /* hipStream_t; NULL = the null stream */
  int64_t sum_seq_lens;      /* optional planning hint: sum of seq_lens (0 = unknown, assume max_seq_len each) */
  /* Optional planning hints (NULL = unknown): host copies of seq_lens [num_seqs] and cu_q_lens [num_seqs + 1]
     holding the same values as the device tables (the caller builds them on the host before uploading; the
     kernels read only the device tables).  A batch whose longest query is prefill-sized runs as two launches
     over all of its sequences, one per class of request (decode-sized: q_len * num_q_heads / num_kv_heads
     <= 32; prefill-sized), each planned for its class, as one scheduler step packs them
     (scheduler.rs:258-271).  With cu_q_lens_host the planner knows the classes (one launch when there is one
     class) and seq_lens_host sizes each class's context split.  Hints only shape the plans: every row is
     computed from the device tables whatever they say, so a stale hint costs speed, not results (with
     MVR_ATTN_CHECKED=true a hint that differs from the device tables is an error).  Read during the call
     only. */
  const int32_t* seq_lens_host;
  const int32_t* cu_q_lens_host;
  /* Token dimension of q and out (0 = unknown; the bindings fill it from q's shape): cu_q_lens[num_seqs] must
     not exceed it, and when given it must lie in [num_seqs, num_seqs * max_q_len].  Without cu_q_lens_host it
     shapes the two launches of a mixed batch: the tokens beyond one per sequence are taken to fill prefill
     requests of max_q_len each packed after the decodes, and a call whose tokens could fill every sequence
     that way runs as one prefill launch.  Checked by mvr_paged_attention_validate against the host
     cu_q_lens and, with MVR_ATTN_CHECKED=true, against the device copy. */
  int32_t total_q;
} mvr_paged_attention_args;

/* Bytes of workspace mvr_paged_attention needs for these arguments (depends
   only on the scalar fields; 0 when no sequence is split into context
   partitions and page_size is a multiple of 16).  The workspace holds fp32
   partial results of the partitions and, when page_size is not a multiple of
   16, a copy of the batch's K/V in 16-token pages (num_seqs x
   ceil(max_seq_len / 16) pages) with its block table; its contents need no
   initialisation and are dead after the call.  Calls that share a workspace
   must not overlap in time. */
size_t mvr_paged_attention_workspace_size(const mvr_paged_attention_args* args);

/* Batched page-wise attention (decode, speculative verification and chunked
   prefill in one entry point).  Replaces forward_paged_attention
   (common.rs:739-817) for every request of a layer in one launch sequence,
   removing the per-request loop of forward_attention (common.rs:285-327).
   Checks the scalar arguments on the host; device tables are trusted (see
   mvr_paged_attention_validate). */
int mvr_paged_attention(const mvr_paged_attention_args* args);

/* Allocation-free variant of mvr_paged_attention.  It has no counterpart in
   the reference: it is for callers that cannot allocate device memory or hand
   over a workspace (code under HIP graph capture, tight serving loops,
   harnesses that forbid hipMalloc).  Same arguments, output and numerics as
   mvr_paged_attention, except that args->workspace and workspace_bytes are
   ignored: the split-context partials (and the 16-token repack of pages that
   a call cannot read in place) live in a static device array of the
   library, MVR_NOALLOC_SCRATCH_BYTES per device, held from the first use on
   that device until the process ends.  A call that needs more returns
   MVR_E_WORKSPACE (use mvr_paged_attention with a workspace for it).  It
   calls no allocator.  Every call on one device shares that device's array:
   calls that overlap in time on one device (other threads or streams) race,
   calls on one stream are ordered.  The array needs no initialisation:
   results never depend on what an earlier call left in it.  MVR_ATTN_CHECKED
   does not apply to it.  The first call on a device looks up the array's
   device address (hipGetSymbolAddress, which may load the library's code
   object): make one call on each device outside any stream capture before
   capturing calls into a graph. */
#define MVR_NOALLOC_SCRATCH_BYTES (64u << 20)
int mvr_paged_attention_noalloc(const mvr_paged_attention_args* args);

/* Host-side checks of the tables the device will read, mirroring the
   reference's errors: seq_len == cached_kv_len + q_len >= q_len >= 1
   (common.rs:447-454), pages covering every length (common.rs:776-781),
   page ids inside the pool.  Host copies of the tables; any may be NULL to
   skip its checks.  Launches nothing. */
int mvr_paged_attention_validate(const mvr_paged_attention_args* args, const int32_t* block_tables_host,
                                 const int32_t* seq_lens_host, const int32_t* cu_q_lens_host);

/* Prefix sharing (cascade attention).  Requests whose block tables start
   with the same physical pages (a cached prefix adopted from the prefix
   index, kv_cache/prefix_index.rs:174-211, request_state.rs:92-103) form a
   group; the members of a group are consecutive sequences of the batch.
   The shared prefix is attended once per group, by all members' query rows
   together, instead of once per member; each member's remaining keys are
   attended separately and the two results are merged exactly (log-sum-exp
   weights).  Groups cover the first sequences of the batch in order (group
   g holds the consecutive sequences whose packed tokens span
   group_cu_q_lens[g] .. group_cu_q_lens[g+1]); a group may have prefix 0
   (its members share nothing), and sequences after the last group have no
   prefix. */
typedef struct mvr_cascade_groups {
  int32_t num_groups;
  int32_t max_group_q_len;           /* >= every group's packed query tokens */
  int32_t max_prefix_len;            /* >= every group's prefix tokens */
  const int32_t* group_cu_q_lens;    /* device [num_groups + 1]: packed-token range of each group's members */
  const int32_t* group_prefix_lens;  /* device [num_groups]: shared tokens, a multiple of page_size (0 allowed)
                                        and <= every member's cached_kv_len; cascade calls need a page_size
                                        that is a multiple of 16 */
  const int32_t* group_block_tables; /* device [num_groups, max_pages_per_seq]: the shared pages */
  const int32_t* seq_prefix_lens;    /* device [num_seqs]: prefix tokens of the sequence's group, 0 if none */
  int64_t sum_prefix_lens;           /* optional planning hint: sum of seq_prefix_lens (0 = unknown) */
} mvr_cascade_groups;

/* Workspace for mvr_paged_attention_cascade (no initialisation needed). */
size_t mvr_paged_attention_cascade_workspace_size(const mvr_paged_attention_args* args,
                                                  const mvr_cascade_groups* groups);

/* mvr_paged_attention with shared prefixes read once per group.  Same
   arguments, output and numerics (an exact split of the softmax sum; results
   differ from the plain call only by rounding).  Stream-ordered, allocates
   nothing.  When the length hints show that the shared reads are a small
   part of the call's key reads (below MVR_ATTN_CASCADE_MIN_SAVING percent,
   default 25), the call runs as mvr_paged_attention instead, which is then
   faster; the workspace size above follows the same choice. */
int mvr_paged_attention_cascade(const mvr_paged_attention_args* args, const mvr_cascade_groups* groups);

/* Host-side checks of the group tables: members consecutive and aligned with
   cu_q_lens, prefix lengths page-aligned and within every member's cached
   tokens, members' first pages equal to the group's pages, seq_prefix_lens
   consistent.  Any pointer may be NULL to skip its checks; launches nothing. */
int mvr_paged_attention_cascade_validate(const mvr_paged_attention_args* args, const mvr_cascade_groups* groups,
                                         const int32_t* block_tables_host, const int32_t* seq_lens_host,
                                         const int32_t* cu_q_lens_host, const int32_t* group_cu_q_lens_host,
                                         const int32_t* group_prefix_lens_host,
                                         const int32_t* group_block_tables_host,
                                         const int32_t* seq_prefix_lens_host);

/* AttentionDimensions (common.rs:189-206). */
typedef struct mvr_attention_dimensions {
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t cached_kv_len;
  int32_t q_len;
} mvr_attention_dimensions;

/* PagedCacheLayout (src/models/mod.rs:94-100) with the page ids already on
   the device as int32. */
typedef struct mvr_paged_cache_layout {
  const void* key_pool;
  const void* value_pool;
  int64_t page_count;
  const int32_t* page_ids; /* device */
  int32_t num_page_ids;
  int32_t per_page_token_count;
  int32_t cached_token_count;
} mvr_paged_cache_layout;

/* Request-level entry with the reference's signature and checks
   (forward_cpu_paged_attention + forward_paged_attention,
   common.rs:426-464 and :739-817): request_q and request_y are
   [1, num_q_heads, q_len, head_dim] contiguous. */
int mvr_forward_paged_attention(int32_t dtype, const mvr_attention_dimensions* dims,
                                const mvr_paged_cache_layout* layout, const void* request_q, void* request_y,
                                void* workspace, size_t workspace_bytes, void* stream);
size_t mvr_forward_paged_attention_workspace_size(int32_t dtype, const mvr_attention_dimensions* dims,
                                                  const mvr_paged_cache_layout* layout);

/* reconstruct_contiguous_tensor (src/model_runner/server/kv_cache/paged_cache.rs:363-391) on the
   device: copies the first cached_token_count tokens of the request's pages
   (page_ids, device int32, logical order) from one pool
   [page_count, 1, num_kv_heads, per_page_token_count, head_dim] into out
   [1, num_kv_heads, cached_token_count, head_dim] contiguous, bit for bit.
   Any page size.  Errors as the reference: an empty cache
   (paged_cache.rs:383-385) and pages that do not cover the length. */
int mvr_reconstruct_contiguous(int32_t dtype, const void* pool, int64_t page_count, int32_t num_kv_heads,
                               int32_t per_page_token_count, int32_t head_dim, const int32_t* page_ids,
                               int32_t num_page_ids, int32_t cached_token_count, void* out, void* stream);

/* RotaryEmbeddingType (common.rs:552-556): Neox rotates dims (i, i + D/2)
   (candle-nn rope), Interleaved rotates (2i, 2i + 1) (candle-nn rope_i). */
typedef enum { MVR_ROPE_NEOX = 0, MVR_ROPE_INTERLEAVED = 1 } mvr_rope_type;

/* The step before attention for every request of a layer: rotary embedding
   of the new Q and K rows and the append of K/V into their page slots.
   Uses the same block tables, seq_lens and cu_q_lens as the attention call
   that follows it: seq_lens counts the tokens after this append, so request
   b's new tokens sit at positions seq_lens[b] - q_len .. seq_lens[b] - 1.
   The block table rows must already hold the pages those positions fall in
   (the host allocates pages; this call only writes). */
typedef struct mvr_rope_append_args {
  int32_t dtype;             /* mvr_dtype */
  int32_t rope_type;         /* mvr_rope_type */
  int32_t num_seqs;
  int32_t num_q_heads;
  int32_t num_kv_heads;      /* divides num_q_heads */
  int32_t head_dim;          /* a multiple of 8, at most 512 */
  int32_t page_size;         /* per_page_token_count, any positive value */
  int64_t num_pages;
  int32_t max_pages_per_seq; /* row stride of block_tables */
  int32_t total_q;           /* packed new tokens = cu_q_lens[num_seqs] (sizes the grid) */
  int32_t max_seq_len;       /* >= every seq_len */
  int32_t rope_len;          /* rows of the cos / sin tables; >= max_seq_len */
  const void* q;             /* [Hq, total_q, D] through strides (elements) */
  int64_t q_stride_head, q_stride_token;
  const void* k;             /* [Hkv, total_q, D] */
  int64_t k_stride_head, k_stride_token;
  const void* v;             /* [Hkv, total_q, D] */
  int64_t v_stride_head, v_stride_token;
  const void* cos_table;     /* [rope_len, D/2] contiguous, activation dtype (RotaryEmbeddingContext::cos) */
  const void* sin_table;     /* [rope_len, D/2] */
  const int32_t* block_tables; /* device */
  const int32_t* seq_lens;     /* device; NULL allowed when num_seqs == 1: seq_len = max_seq_len */
  const int32_t* cu_q_lens;    /* device; NULL allowed when num_seqs == 1: q_len = total_q */
  void* q_out;               /* rotated queries; may be q itself (in place) */
  int64_t q_out_stride_head, q_out_stride_token;
  void* key_pool;            /* written: rotated keys */
  void* value_pool;          /* written: values */
  void* stream;              /* hipStream_t */
} mvr_rope_append_args;

/* forward_rope for Q and K (common.rs:294-307, :344-359) and
   append_new_key_value (kv_cache/paged_cache.rs:170-199, :290-327;
   physical_page_pool.rs:188-209) fused into one launch over every request
   (replaces the per-request part of forward_attention's loop,
   common.rs:285-320).  Arithmetic in the activation dtype with each product
   and sum rounded as the reference's rope kernels do.  Stream-ordered;
   allocates nothing; device tables are trusted (see
   mvr_rope_append_validate). */
int mvr_rope_append(const mvr_rope_append_args* args);

/* Host-side checks of the tables the append will use, mirroring the
   reference's errors: every q_len >= 1 ("cannot append an empty KV-cache
   tensor", kv_cache/utils.rs:33-36), seq_len >= q_len, pages covering every
   position written, page ids inside the pool, no page written by two
   requests, positions inside the rotary tables, and, when page_writable_host
   (one byte per pool page, nonzero = PendingWrite) is given, that every page
   written is writable ("cannot mutate written physical page N",
   physical_page_pool.rs:197-201).  Launches nothing. */
int mvr_rope_append_validate(const mvr_rope_append_args* args, const int32_t* block_tables_host,
                             const int32_t* seq_lens_host, const int32_t* cu_q_lens_host,
                             const uint8_t* page_writable_host);

/* Thread-local description of the last error on this thread ("" if none). */
const char* mvr_last_error(void);

int mvr_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MVR_ATTN_H */
