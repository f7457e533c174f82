// Rust binding of libmvr_attn.so (C ABI: include/mvr_attn.h, ABI version 2).
//
// Drop-in module for lun0522/mini-vllm-rs: copy to src/models/backends/mvr_attn.rs,
// declare it next to the other backend modules (src/models/backends/mod.rs), and
// link the library from build.rs (see build_rs_fragment.rs beside this file).
// The dispatcher branch that calls it goes ahead of forward_cpu_paged_attention
// in forward_self_attention (src/models/backends/common.rs:375-379); with the
// batched entry points it moves up into forward_attention and replaces the
// per-request loop and the cat (common.rs:285-327).
//
// Every #[repr(C)] struct below lists the fields of its C struct in the same
// order with the same widths; every extern fn has the C prototype's argument
// types.  A CPU test of this repository (tests/test_rust_binding.py) parses
// this file and the header and checks both.
#![allow(dead_code)]

use std::ffi::{c_char, c_int, c_void, CStr};

pub const MVR_ATTN_ABI_VERSION: c_int = 3;
pub const MVR_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

// ActivationDType (src/model_runner/mod.rs:331-351).
pub const MVR_DTYPE_F32: i32 = 0;
pub const MVR_DTYPE_F16: i32 = 1;

// RotaryEmbeddingType (common.rs:552-556).
pub const MVR_ROPE_NEOX: i32 = 0;
pub const MVR_ROPE_INTERLEAVED: i32 = 1;

pub const MVR_OK: c_int = 0;
pub const MVR_E_INVALID_ARGUMENT: c_int = -1;
pub const MVR_E_UNSUPPORTED: c_int = -2;
pub const MVR_E_LENGTH_MISMATCH: c_int = -3; // common.rs:447-454
pub const MVR_E_PAGES_UNCOVERED: c_int = -4; // common.rs:776-781
pub const MVR_E_PAGE_ID: c_int = -5;
pub const MVR_E_WORKSPACE: c_int = -6;
pub const MVR_E_HIP: c_int = -7;
pub const MVR_E_READ_ONLY_PAGE: c_int = -8; // physical_page_pool.rs:197-201

#[repr(C)]
pub struct MvrPagedAttentionArgs {
    pub dtype: i32,             // MVR_DTYPE_*
    pub num_seqs: i32,          // requests packed in the call
    pub num_q_heads: i32,
    pub num_kv_heads: i32,
    pub head_dim: i32,          // a multiple of 32 in [32, 256]
    pub page_size: i32,         // per_page_token_count
    pub num_pages: i64,         // page_count of each pool
    pub max_pages_per_seq: i32, // row stride of block_tables
    pub max_q_len: i32,
    pub max_seq_len: i32,
    pub scale: f32,             // 0.0: 1/sqrt(head_dim), as common.rs:784-785
    pub q: *const c_void,       // [1, Hq, packed_q_len, D] after RoPE (common.rs:268-275)
    pub q_stride_head: i64,
    pub q_stride_token: i64,
    pub key_pool: *const c_void, // PagedCacheLayout::key_pool [N, 1, Hkv, P, D] (src/models/mod.rs:94-100)
    pub value_pool: *const c_void,
    pub block_tables: *const i32, // device int32 [num_seqs, max_pages_per_seq]: page_ids per request
    pub seq_lens: *const i32,     // device: cached_token_count per request
    pub cu_q_lens: *const i32,    // device: q_start_index prefix sums (common.rs:603-626)
    pub out: *mut c_void,         // [1, Hq, packed_q_len, D]
    pub out_stride_head: i64,
    pub out_stride_token: i64,
    pub workspace: *mut c_void,
    pub workspace_bytes: usize,
    pub stream: *mut c_void,      // hipStream_t
    pub sum_seq_lens: i64,        // optional hint: sum of seq_lens (0 = unknown)
    pub seq_lens_host: *const i32, // optional hint: host copy of seq_lens (null = unknown)
    pub cu_q_lens_host: *const i32, // optional hint: host copy of cu_q_lens (null = unknown)
    pub total_q: i32,               // token dimension of q and out (0 = unknown): bounds cu_q_lens[num_seqs]
}

#[repr(C)]
pub struct MvrCascadeGroups {
    pub num_groups: i32,
    pub max_group_q_len: i32,
    pub max_prefix_len: i32,
    pub group_cu_q_lens: *const i32,    // device [num_groups + 1]
    pub group_prefix_lens: *const i32,  // device [num_groups], multiples of per_page_token_count
    pub group_block_tables: *const i32, // device [num_groups, max_pages_per_seq]
    pub seq_prefix_lens: *const i32,    // device [num_seqs]
    pub sum_prefix_lens: i64,           // optional hint (0 = unknown)
}

// AttentionDimensions (common.rs:189-206).
#[repr(C)]
pub struct MvrAttentionDimensions {
    pub num_q_heads: i32,
    pub num_kv_heads: i32,
    pub head_dim: i32,
    pub cached_kv_len: i32,
    pub q_len: i32,
}

// PagedCacheLayout (src/models/mod.rs:94-100) with page_ids uploaded as int32.
#[repr(C)]
pub struct MvrPagedCacheLayout {
    pub key_pool: *const c_void,
    pub value_pool: *const c_void,
    pub page_count: i64,
    pub page_ids: *const i32,
    pub num_page_ids: i32,
    pub per_page_token_count: i32,
    pub cached_token_count: i32,
}

#[repr(C)]
pub struct MvrRopeAppendArgs {
    pub dtype: i32,
    pub rope_type: i32, // MVR_ROPE_*
    pub num_seqs: i32,
    pub num_q_heads: i32,
    pub num_kv_heads: i32,
    pub head_dim: i32,
    pub page_size: i32,
    pub num_pages: i64,
    pub max_pages_per_seq: i32,
    pub total_q: i32,   // packed_q_len
    pub max_seq_len: i32,
    pub rope_len: i32,  // rows of RotaryEmbeddingContext::cos / sin
    pub q: *const c_void,
    pub q_stride_head: i64,
    pub q_stride_token: i64,
    pub k: *const c_void,
    pub k_stride_head: i64,
    pub k_stride_token: i64,
    pub v: *const c_void,
    pub v_stride_head: i64,
    pub v_stride_token: i64,
    pub cos_table: *const c_void,
    pub sin_table: *const c_void,
    pub block_tables: *const i32,
    pub seq_lens: *const i32,
    pub cu_q_lens: *const i32,
    pub q_out: *mut c_void,
    pub q_out_stride_head: i64,
    pub q_out_stride_token: i64,
    pub key_pool: *mut c_void,
    pub value_pool: *mut c_void,
    pub stream: *mut c_void,
}

extern "C" {
    pub fn mvr_paged_attention_workspace_size(args: *const MvrPagedAttentionArgs) -> usize;
    pub fn mvr_paged_attention(args: *const MvrPagedAttentionArgs) -> c_int;
    pub fn mvr_paged_attention_noalloc(args: *const MvrPagedAttentionArgs) -> c_int;
    pub fn mvr_paged_attention_validate(args: *const MvrPagedAttentionArgs, block_tables_host: *const i32,
                                        seq_lens_host: *const i32, cu_q_lens_host: *const i32) -> c_int;
    pub fn mvr_paged_attention_cascade_workspace_size(args: *const MvrPagedAttentionArgs,
                                                      groups: *const MvrCascadeGroups) -> usize;
    pub fn mvr_paged_attention_cascade(args: *const MvrPagedAttentionArgs, groups: *const MvrCascadeGroups) -> c_int;
    pub fn mvr_paged_attention_cascade_validate(args: *const MvrPagedAttentionArgs, groups: *const MvrCascadeGroups,
                                                block_tables_host: *const i32, seq_lens_host: *const i32,
                                                cu_q_lens_host: *const i32, group_cu_q_lens_host: *const i32,
                                                group_prefix_lens_host: *const i32,
                                                group_block_tables_host: *const i32,
                                                seq_prefix_lens_host: *const i32) -> c_int;
    pub fn mvr_forward_paged_attention(dtype: i32, dims: *const MvrAttentionDimensions,
                                       layout: *const MvrPagedCacheLayout, request_q: *const c_void,
                                       request_y: *mut c_void, workspace: *mut c_void, workspace_bytes: usize,
                                       stream: *mut c_void) -> c_int;
    pub fn mvr_forward_paged_attention_workspace_size(dtype: i32, dims: *const MvrAttentionDimensions,
                                                      layout: *const MvrPagedCacheLayout) -> usize;
    pub fn mvr_reconstruct_contiguous(dtype: i32, pool: *const c_void, page_count: i64, num_kv_heads: i32,
                                      per_page_token_count: i32, head_dim: i32, page_ids: *const i32,
                                      num_page_ids: i32, cached_token_count: i32, out: *mut c_void,
                                      stream: *mut c_void) -> c_int;
    pub fn mvr_rope_append(args: *const MvrRopeAppendArgs) -> c_int;
    pub fn mvr_rope_append_validate(args: *const MvrRopeAppendArgs, block_tables_host: *const i32,
                                    seq_lens_host: *const i32, cu_q_lens_host: *const i32,
                                    page_writable_host: *const u8) -> c_int;
    pub fn mvr_last_error() -> *const c_char;
    pub fn mvr_abi_version() -> c_int;
}

/// The library's message for a failed call, as candle_core::bail! would carry it.
fn check(rc: c_int) -> candle_core::Result<()> {
    if rc == MVR_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(mvr_last_error()) }.to_string_lossy().into_owned();
    candle_core::bail!("{msg} (mvr_attn error {rc})")
}

/// Refuses a library built for another ABI (call once when the backend starts).
pub fn check_abi() -> candle_core::Result<()> {
    let v = unsafe { mvr_abi_version() };
    if v != MVR_ATTN_ABI_VERSION {
        candle_core::bail!("libmvr_attn.so has ABI version {v}, this binding expects {MVR_ATTN_ABI_VERSION}");
    }
    Ok(())
}

pub fn workspace_size(args: &MvrPagedAttentionArgs) -> usize {
    unsafe { mvr_paged_attention_workspace_size(args) }
}

/// forward_paged_attention for every request of a layer (common.rs:739-817 batched over common.rs:285-327).
pub fn paged_attention(args: &MvrPagedAttentionArgs) -> candle_core::Result<()> {
    check(unsafe { mvr_paged_attention(args) })
}

/// paged_attention without a workspace: the library's static device scratch (MVR_NOALLOC_SCRATCH_BYTES per
/// device) holds the partials, for callers that cannot allocate (graph capture, fixed serving loops).
/// Calls that overlap in time on one device race on that scratch.
pub fn paged_attention_noalloc(args: &MvrPagedAttentionArgs) -> candle_core::Result<()> {
    check(unsafe { mvr_paged_attention_noalloc(args) })
}

/// The checks of common.rs:447-454 and :776-781 on host copies of the tables (no launch).  The slices must hold
/// the whole tables the arguments describe (the library reads that many entries), else this returns an error
/// without calling it.
pub fn validate(args: &MvrPagedAttentionArgs, block_tables: &[i32], seq_lens: &[i32], cu_q_lens: &[i32])
    -> candle_core::Result<()> {
    let n = args.num_seqs.max(0) as usize;
    let pages = n.saturating_mul(args.max_pages_per_seq.max(0) as usize);
    if block_tables.len() < pages || seq_lens.len() < n || cu_q_lens.len() < n + 1 {
        candle_core::bail!(
            "validate: tables shorter than the arguments describe (block_tables {} < {}, seq_lens {} < {} or \
             cu_q_lens {} < {})",
            block_tables.len(), pages, seq_lens.len(), n, cu_q_lens.len(), n + 1
        );
    }
    check(unsafe { mvr_paged_attention_validate(args, block_tables.as_ptr(), seq_lens.as_ptr(), cu_q_lens.as_ptr()) })
}

pub fn cascade_workspace_size(args: &MvrPagedAttentionArgs, groups: &MvrCascadeGroups) -> usize {
    unsafe { mvr_paged_attention_cascade_workspace_size(args, groups) }
}

/// paged_attention with each group's adopted prefix (prefix_index.rs:174-211) attended once.
pub fn paged_attention_cascade(args: &MvrPagedAttentionArgs, groups: &MvrCascadeGroups) -> candle_core::Result<()> {
    check(unsafe { mvr_paged_attention_cascade(args, groups) })
}

/// forward_cpu_paged_attention + forward_paged_attention for one request (common.rs:426-464, :739-817).
pub fn forward_paged_attention(dtype: i32, dims: &MvrAttentionDimensions, layout: &MvrPagedCacheLayout,
                               request_q: *const c_void, request_y: *mut c_void, workspace: *mut c_void,
                               workspace_bytes: usize, stream: *mut c_void) -> candle_core::Result<()> {
    check(unsafe { mvr_forward_paged_attention(dtype, dims, layout, request_q, request_y, workspace, workspace_bytes, stream) })
}

/// forward_rope on Q and K plus append_new_key_value for every request of a layer (common.rs:294-320).
pub fn rope_append(args: &MvrRopeAppendArgs) -> candle_core::Result<()> {
    check(unsafe { mvr_rope_append(args) })
}

/// reconstruct_contiguous_tensor for one pool on the device (paged_cache.rs:363-391).
pub fn reconstruct_contiguous(dtype: i32, pool: *const c_void, page_count: i64, num_kv_heads: i32,
                              per_page_token_count: i32, head_dim: i32, page_ids: *const i32, num_page_ids: i32,
                              cached_token_count: i32, out: *mut c_void, stream: *mut c_void)
    -> candle_core::Result<()> {
    check(unsafe {
        mvr_reconstruct_contiguous(dtype, pool, page_count, num_kv_heads, per_page_token_count, head_dim, page_ids,
                                   num_page_ids, cached_token_count, out, stream)
    })
}
