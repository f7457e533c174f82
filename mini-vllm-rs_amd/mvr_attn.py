"""Python binding of libmvr_attn.so (C ABI in include/mvr_attn.h).

Mirrors the reference's attention entry points:
  * paged_attention(...)          batched page-wise attention over one layer's
                                  packed requests (replaces the per-request
                                  loop of forward_attention, common.rs:285-327);
  * forward_paged_attention(...)  one request with a PagedCacheLayout, same
                                  arguments and errors as forward_paged_attention
                                  (common.rs:739-817) behind
                                  forward_cpu_paged_attention (common.rs:426-464);
  * rope_append(...)              RoPE of the new Q/K rows and the KV-page append
                                  for every request of a layer (common.rs:294-320,
                                  kv_cache/paged_cache.rs:290-327);
  * reconstruct_contiguous(...)   reconstruct_contiguous_tensor
                                  (kv_cache/paged_cache.rs:363-391).
Tensors are torch tensors on the GPU; torch supplies device memory and the
current stream only.  The library must be built (make -C mini-vllm-rs_amd):
there is no CPU fallback, and a missing library raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import math
import os
from dataclasses import dataclass
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmvr_attn.so")

ABI_VERSION = 3  # MVR_ATTN_ABI_VERSION of include/mvr_attn.h

DTYPE_F32, DTYPE_F16 = 0, 1

MVR_OK = 0
MVR_E_INVALID_ARGUMENT = -1
MVR_E_UNSUPPORTED = -2
MVR_E_LENGTH_MISMATCH = -3
MVR_E_PAGES_UNCOVERED = -4
MVR_E_PAGE_ID = -5
MVR_E_WORKSPACE = -6
MVR_E_HIP = -7
MVR_E_READ_ONLY_PAGE = -8

ROPE_NEOX, ROPE_INTERLEAVED = 0, 1

EXPORTED_SYMBOLS = (
    "mvr_abi_version",
    "mvr_last_error",
    "mvr_paged_attention",
    "mvr_paged_attention_workspace_size",
    "mvr_paged_attention_validate",
    "mvr_forward_paged_attention",
    "mvr_forward_paged_attention_workspace_size",
    "mvr_reconstruct_contiguous",
    "mvr_rope_append",
    "mvr_rope_append_validate",
    "mvr_paged_attention_cascade",
    "mvr_paged_attention_cascade_workspace_size",
    "mvr_paged_attention_cascade_validate",
    "mvr_paged_attention_noalloc",
)

NOALLOC_SCRATCH_BYTES = 64 << 20  # MVR_NOALLOC_SCRATCH_BYTES of include/mvr_attn.h


class MvrError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{message} (code {code})")
        self.code = code
        self.message = message


class PagedAttentionArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("num_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int64),
        ("max_pages_per_seq", ctypes.c_int32),
        ("max_q_len", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q", ctypes.c_void_p),
        ("q_stride_head", ctypes.c_int64),
        ("q_stride_token", ctypes.c_int64),
        ("key_pool", ctypes.c_void_p),
        ("value_pool", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("cu_q_lens", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("out_stride_head", ctypes.c_int64),
        ("out_stride_token", ctypes.c_int64),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("stream", ctypes.c_void_p),
        ("sum_seq_lens", ctypes.c_int64),
        ("seq_lens_host", ctypes.c_void_p),
        ("cu_q_lens_host", ctypes.c_void_p),
        ("total_q", ctypes.c_int32),
    ]


class AttentionDimensions(ctypes.Structure):
    _fields_ = [
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("cached_kv_len", ctypes.c_int32),
        ("q_len", ctypes.c_int32),
    ]


class PagedCacheLayoutC(ctypes.Structure):
    _fields_ = [
        ("key_pool", ctypes.c_void_p),
        ("value_pool", ctypes.c_void_p),
        ("page_count", ctypes.c_int64),
        ("page_ids", ctypes.c_void_p),
        ("num_page_ids", ctypes.c_int32),
        ("per_page_token_count", ctypes.c_int32),
        ("cached_token_count", ctypes.c_int32),
    ]


class CascadeGroups(ctypes.Structure):
    _fields_ = [
        ("num_groups", ctypes.c_int32),
        ("max_group_q_len", ctypes.c_int32),
        ("max_prefix_len", ctypes.c_int32),
        ("group_cu_q_lens", ctypes.c_void_p),
        ("group_prefix_lens", ctypes.c_void_p),
        ("group_block_tables", ctypes.c_void_p),
        ("seq_prefix_lens", ctypes.c_void_p),
        ("sum_prefix_lens", ctypes.c_int64),
    ]


class RopeAppendArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("rope_type", ctypes.c_int32),
        ("num_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int64),
        ("max_pages_per_seq", ctypes.c_int32),
        ("total_q", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("rope_len", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("q_stride_head", ctypes.c_int64),
        ("q_stride_token", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("k_stride_head", ctypes.c_int64),
        ("k_stride_token", ctypes.c_int64),
        ("v", ctypes.c_void_p),
        ("v_stride_head", ctypes.c_int64),
        ("v_stride_token", ctypes.c_int64),
        ("cos_table", ctypes.c_void_p),
        ("sin_table", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("cu_q_lens", ctypes.c_void_p),
        ("q_out", ctypes.c_void_p),
        ("q_out_stride_head", ctypes.c_int64),
        ("q_out_stride_token", ctypes.c_int64),
        ("key_pool", ctypes.c_void_p),
        ("value_pool", ctypes.c_void_p),
        ("stream", ctypes.c_void_p),
    ]


_lib = None


def library_path() -> str:
    return LIB_PATH


def load_library():
    """Loads libmvr_attn.so from this package directory; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` (no CPU fallback exists)")
    lib = ctypes.CDLL(LIB_PATH)
    lib.mvr_abi_version.restype = ctypes.c_int
    lib.mvr_last_error.restype = ctypes.c_char_p
    lib.mvr_paged_attention.restype = ctypes.c_int
    lib.mvr_paged_attention.argtypes = [ctypes.POINTER(PagedAttentionArgs)]
    lib.mvr_paged_attention_noalloc.restype = ctypes.c_int
    lib.mvr_paged_attention_noalloc.argtypes = [ctypes.POINTER(PagedAttentionArgs)]
    lib.mvr_paged_attention_workspace_size.restype = ctypes.c_size_t
    lib.mvr_paged_attention_workspace_size.argtypes = [ctypes.POINTER(PagedAttentionArgs)]
    lib.mvr_paged_attention_validate.restype = ctypes.c_int
    lib.mvr_paged_attention_validate.argtypes = [ctypes.POINTER(PagedAttentionArgs), ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.c_void_p]
    lib.mvr_forward_paged_attention.restype = ctypes.c_int
    lib.mvr_forward_paged_attention.argtypes = [ctypes.c_int32, ctypes.POINTER(AttentionDimensions),
                                                ctypes.POINTER(PagedCacheLayoutC), ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.mvr_forward_paged_attention_workspace_size.restype = ctypes.c_size_t
    lib.mvr_forward_paged_attention_workspace_size.argtypes = [ctypes.c_int32, ctypes.POINTER(AttentionDimensions),
                                                               ctypes.POINTER(PagedCacheLayoutC)]
    lib.mvr_reconstruct_contiguous.restype = ctypes.c_int
    lib.mvr_reconstruct_contiguous.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                               ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                               ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    lib.mvr_rope_append.restype = ctypes.c_int
    lib.mvr_rope_append.argtypes = [ctypes.POINTER(RopeAppendArgs)]
    lib.mvr_rope_append_validate.restype = ctypes.c_int
    lib.mvr_rope_append_validate.argtypes = [ctypes.POINTER(RopeAppendArgs), ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_void_p, ctypes.c_void_p]
    lib.mvr_paged_attention_cascade.restype = ctypes.c_int
    lib.mvr_paged_attention_cascade.argtypes = [ctypes.POINTER(PagedAttentionArgs), ctypes.POINTER(CascadeGroups)]
    lib.mvr_paged_attention_cascade_workspace_size.restype = ctypes.c_size_t
    lib.mvr_paged_attention_cascade_workspace_size.argtypes = [ctypes.POINTER(PagedAttentionArgs),
                                                               ctypes.POINTER(CascadeGroups)]
    lib.mvr_paged_attention_cascade_validate.restype = ctypes.c_int
    lib.mvr_paged_attention_cascade_validate.argtypes = [ctypes.POINTER(PagedAttentionArgs),
                                                         ctypes.POINTER(CascadeGroups)] + [ctypes.c_void_p] * 7
    if lib.mvr_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libmvr_attn.so ABI version {lib.mvr_abi_version()}, this binding is {ABI_VERSION}")
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != MVR_OK:
        msg = load_library().mvr_last_error().decode()
        raise MvrError(rc, msg)


def _torch():
    import torch  # imported lazily: CPU-only users of this module need no torch

    return torch


def dtype_code(t) -> int:
    torch = _torch()
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.float32:
        return DTYPE_F32
    raise MvrError(MVR_E_UNSUPPORTED, f"activation dtype {t.dtype} is not F32 or F16")


def _stream_handle(stream) -> Optional[int]:
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _stream_scope(stream, *tensors):
    """Scope of one call launched on `stream`.  When that is not the current stream, the call's own
    allocations (output, workspace) are made inside torch.cuda.stream(stream), so the caching allocator
    hands their blocks to later work only in that stream's order, and every device tensor the kernels
    read or write is recorded on `stream`, so that freeing it on its own stream before the kernels ran
    cannot let another allocation reuse its memory meanwhile."""
    torch = _torch()
    if stream is None or stream == torch.cuda.current_stream():
        return contextlib.nullcontext()
    for t in tensors:
        if t is not None and getattr(t, "is_cuda", False):
            t.record_stream(stream)
    return torch.cuda.stream(stream)


def _host_int32(x):
    """A contiguous int32 numpy copy of a host table (or None)."""
    if x is None:
        return None
    import numpy as np

    return np.ascontiguousarray(x, dtype=np.int32)


def make_args(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, *, max_q_len: int,
              max_seq_len: int, scale: float = 0.0, stream=None, sum_seq_lens: int = 0, seq_lens_host=None,
              cu_q_lens_host=None) -> PagedAttentionArgs:
    """Fills the C argument struct.  q / out: [Hq, total_q, D] (last dim contiguous);
    pools: [num_pages, 1, Hkv, page_size, D]; block_tables int32 [num_seqs, max_pages].
    seq_lens_host / cu_q_lens_host: optional host copies of the two length tables (planning hints: with them a
    batch mixing decode-sized and prefill-sized requests runs each class on its own launch)."""
    n_pages, one, hkv, page_size, d = key_pool.shape
    if one != 1 or value_pool.shape != key_pool.shape:
        raise MvrError(MVR_E_INVALID_ARGUMENT, "pools must be [num_pages, 1, num_kv_heads, page_size, head_dim]")
    if q.dim() != 3 or q.stride(2) != 1 or out.dim() != 3 or out.stride(2) != 1:
        raise MvrError(MVR_E_INVALID_ARGUMENT, "q and out must be [num_q_heads, tokens, head_dim] with unit last stride")
    if not key_pool.is_contiguous() or not value_pool.is_contiguous() or not block_tables.is_contiguous():
        raise MvrError(MVR_E_INVALID_ARGUMENT, "pools and block tables must be contiguous")
    a = PagedAttentionArgs()
    a.dtype = dtype_code(q)
    a.num_seqs = block_tables.shape[0]
    a.num_q_heads = q.shape[0]
    a.num_kv_heads = hkv
    a.head_dim = d
    a.page_size = page_size
    a.num_pages = n_pages
    a.max_pages_per_seq = block_tables.shape[1]
    a.max_q_len = max_q_len
    a.max_seq_len = max_seq_len
    a.scale = scale
    a.q = q.data_ptr()
    a.q_stride_head = q.stride(0)
    a.q_stride_token = q.stride(1)
    a.key_pool = key_pool.data_ptr()
    a.value_pool = value_pool.data_ptr()
    a.block_tables = block_tables.data_ptr()
    a.seq_lens = seq_lens.data_ptr() if seq_lens is not None else None
    a.cu_q_lens = cu_q_lens.data_ptr() if cu_q_lens is not None else None
    a.out = out.data_ptr()
    a.out_stride_head = out.stride(0)
    a.out_stride_token = out.stride(1)
    a.stream = _stream_handle(stream)
    a.sum_seq_lens = int(sum_seq_lens)
    a.total_q = q.shape[1]
    sl_h, cu_h = _host_int32(seq_lens_host), _host_int32(cu_q_lens_host)
    if sl_h is not None and sl_h.shape != (a.num_seqs,):
        raise MvrError(MVR_E_INVALID_ARGUMENT, "seq_lens_host must hold num_seqs entries")
    if cu_h is not None and cu_h.shape != (a.num_seqs + 1,):
        raise MvrError(MVR_E_INVALID_ARGUMENT, "cu_q_lens_host must hold num_seqs + 1 entries")
    a.seq_lens_host = sl_h.ctypes.data if sl_h is not None else None
    a.cu_q_lens_host = cu_h.ctypes.data if cu_h is not None else None
    # The struct holds raw device addresses: keep the tensors alive with it, so that a table built inline
    # (make_args(..., torch.tensor(...).cuda(), ...)) is not freed and its memory reused before the launch.
    a._keep = (q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, sl_h, cu_h)
    return a


def workspace_size(args: PagedAttentionArgs) -> int:
    return int(load_library().mvr_paged_attention_workspace_size(ctypes.byref(args)))


def new_workspace(nbytes: int, device):
    """Device scratch for context-partition partials, and for the 16-token repack of pages that a call cannot
    read in place (no initialisation needed)."""
    return _torch().empty(max(int(nbytes), 256), dtype=_torch().uint8, device=device)


def paged_attention(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out=None, *, max_q_len: int,
                    max_seq_len: int, scale: float = 0.0, workspace=None, stream=None, sum_seq_lens: int = 0,
                    seq_lens_host=None, cu_q_lens_host=None):
    """Batched page-wise attention; returns out [Hq, total_q, D] in q's dtype."""
    torch = _torch()
    with _stream_scope(stream, q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, workspace):
        if out is None:
            out = torch.empty_like(q, memory_format=torch.contiguous_format)
        a = make_args(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, max_q_len=max_q_len,
                      max_seq_len=max_seq_len, scale=scale, stream=stream, sum_seq_lens=sum_seq_lens,
                      seq_lens_host=seq_lens_host, cu_q_lens_host=cu_q_lens_host)
        need = workspace_size(a)
        if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
            workspace = new_workspace(need, q.device)
        if workspace is not None:
            a.workspace = workspace.data_ptr()
            a.workspace_bytes = workspace.numel() * workspace.element_size()
        _check(load_library().mvr_paged_attention(ctypes.byref(a)))
    return out


def paged_attention_noalloc(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, *, max_q_len: int,
                            max_seq_len: int, scale: float = 0.0, stream=None, sum_seq_lens: int = 0,
                            seq_lens_host=None, cu_q_lens_host=None):
    """mvr_paged_attention_noalloc: the caller passes the output; the library's static device scratch replaces
    the workspace, so nothing is allocated (calls that overlap in time on one device race on that scratch)."""
    with _stream_scope(stream, q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out):
        a = make_args(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, max_q_len=max_q_len,
                      max_seq_len=max_seq_len, scale=scale, stream=stream, sum_seq_lens=sum_seq_lens,
                      seq_lens_host=seq_lens_host, cu_q_lens_host=cu_q_lens_host)
        _check(load_library().mvr_paged_attention_noalloc(ctypes.byref(a)))
    return out


def validate(args: PagedAttentionArgs, block_tables_host=None, seq_lens_host=None, cu_q_lens_host=None) -> None:
    """Host-side table checks (numpy int32 arrays or None); raises MvrError."""
    import numpy as np

    def ptr(x):
        if x is None:
            return None
        x = np.ascontiguousarray(x, dtype=np.int32)
        ptr.keep.append(x)
        return x.ctypes.data

    ptr.keep = []
    _check(load_library().mvr_paged_attention_validate(ctypes.byref(args), ptr(block_tables_host),
                                                      ptr(seq_lens_host), ptr(cu_q_lens_host)))


@dataclass
class PagedCacheLayout:
    """PagedCacheLayout (src/models/mod.rs:94-100); page_ids live on the device as int32."""

    key_pool: object
    value_pool: object
    page_ids: object
    per_page_token_count: int
    cached_token_count: int


def forward_paged_attention(request_q, layout: PagedCacheLayout, num_q_heads: int, num_kv_heads: int, head_dim: int,
                            cached_kv_len: int, q_len: int, stream=None):
    """One request: request_q [1, Hq, q_len, D] -> [1, Hq, q_len, D] (common.rs:739-817)."""
    torch = _torch()
    dims = AttentionDimensions(num_q_heads, num_kv_heads, head_dim, cached_kv_len, q_len)
    c = PagedCacheLayoutC(layout.key_pool.data_ptr(), layout.value_pool.data_ptr(), layout.key_pool.shape[0],
                          layout.page_ids.data_ptr(), layout.page_ids.numel(), layout.per_page_token_count,
                          layout.cached_token_count)
    with _stream_scope(stream, request_q, layout.key_pool, layout.value_pool, layout.page_ids):
        q = request_q.contiguous()
        y = torch.empty_like(q)
        dt = dtype_code(q)
        lib = load_library()
        need = int(lib.mvr_forward_paged_attention_workspace_size(dt, ctypes.byref(dims), ctypes.byref(c)))
        ws = new_workspace(need, q.device)
        _check(lib.mvr_forward_paged_attention(dt, ctypes.byref(dims), ctypes.byref(c), q.data_ptr(), y.data_ptr(),
                                               ws.data_ptr(), need, _stream_handle(stream)))
    return y


def reconstruct_contiguous(pool, page_ids, cached_token_count: int, stream=None):
    """reconstruct_contiguous_tensor (paged_cache.rs:363-391): pool [N, 1, Hkv, P, D], page_ids int32 (device)
    -> [1, Hkv, cached_token_count, D], bit-exact."""
    torch = _torch()
    n, _, hkv, page_size, d = pool.shape
    with _stream_scope(stream, pool, page_ids):
        out = torch.empty((1, hkv, max(int(cached_token_count), 0), d), dtype=pool.dtype, device=pool.device)
        rc = load_library().mvr_reconstruct_contiguous(dtype_code(pool), pool.data_ptr(), n, hkv, page_size, d,
                                                       page_ids.data_ptr(), page_ids.numel(), int(cached_token_count),
                                                       out.data_ptr(), _stream_handle(stream))
    _check(rc)
    return out


def pages_for(seq_len: int, page_size: int) -> int:
    return math.ceil(seq_len / page_size)


def make_rope_append_args(q, k, v, cos_table, sin_table, block_tables, seq_lens, cu_q_lens, key_pool, value_pool,
                          q_out, *, max_seq_len: int, rope_type: int = ROPE_NEOX, stream=None) -> RopeAppendArgs:
    """q / q_out [Hq, total_q, D], k / v [Hkv, total_q, D] (unit last stride); cos / sin [rope_len, D/2];
    pools [num_pages, 1, Hkv, page_size, D]; tables as for paged_attention (seq_lens after the append)."""
    n_pages, one, hkv, page_size, d = key_pool.shape
    if one != 1 or value_pool.shape != key_pool.shape:
        raise MvrError(MVR_E_INVALID_ARGUMENT, "pools must be [num_pages, 1, num_kv_heads, page_size, head_dim]")
    for t in (q, k, v, q_out):
        if t.dim() != 3 or t.stride(2) != 1:
            raise MvrError(MVR_E_INVALID_ARGUMENT, "q, k, v and q_out must be [heads, tokens, head_dim], unit last stride")
    if not (key_pool.is_contiguous() and value_pool.is_contiguous() and block_tables.is_contiguous()
            and cos_table.is_contiguous() and sin_table.is_contiguous()):
        raise MvrError(MVR_E_INVALID_ARGUMENT, "pools, tables and cos/sin must be contiguous")
    a = RopeAppendArgs()
    a.dtype = dtype_code(q)
    a.rope_type = rope_type
    a.num_seqs = block_tables.shape[0]
    a.num_q_heads = q.shape[0]
    a.num_kv_heads = hkv
    a.head_dim = d
    a.page_size = page_size
    a.num_pages = n_pages
    a.max_pages_per_seq = block_tables.shape[1]
    a.total_q = q.shape[1]
    a.max_seq_len = max_seq_len
    a.rope_len = cos_table.shape[0]
    a.q, a.q_stride_head, a.q_stride_token = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_stride_head, a.k_stride_token = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_stride_head, a.v_stride_token = v.data_ptr(), v.stride(0), v.stride(1)
    a.cos_table = cos_table.data_ptr()
    a.sin_table = sin_table.data_ptr()
    a.block_tables = block_tables.data_ptr()
    a.seq_lens = seq_lens.data_ptr() if seq_lens is not None else None
    a.cu_q_lens = cu_q_lens.data_ptr() if cu_q_lens is not None else None
    a.q_out, a.q_out_stride_head, a.q_out_stride_token = q_out.data_ptr(), q_out.stride(0), q_out.stride(1)
    a.key_pool = key_pool.data_ptr()
    a.value_pool = value_pool.data_ptr()
    a.stream = _stream_handle(stream)
    a._keep = (q, k, v, cos_table, sin_table, block_tables, seq_lens, cu_q_lens, q_out, key_pool, value_pool)
    return a


def rope_append(q, k, v, cos_table, sin_table, block_tables, seq_lens, cu_q_lens, key_pool, value_pool, q_out=None,
                *, max_seq_len: int, rope_type: int = ROPE_NEOX, stream=None):
    """Rotates q into q_out (a new tensor unless given; may be q itself) and writes the rotated k and v into
    their page slots; returns q_out."""
    torch = _torch()
    with _stream_scope(stream, q, k, v, cos_table, sin_table, block_tables, seq_lens, cu_q_lens, key_pool,
                       value_pool, q_out):
        if q_out is None:
            q_out = torch.empty_like(q, memory_format=torch.contiguous_format)
        a = make_rope_append_args(q, k, v, cos_table, sin_table, block_tables, seq_lens, cu_q_lens, key_pool,
                                  value_pool, q_out, max_seq_len=max_seq_len, rope_type=rope_type, stream=stream)
        _check(load_library().mvr_rope_append(ctypes.byref(a)))
    return q_out


def validate_rope_append(args: RopeAppendArgs, block_tables_host=None, seq_lens_host=None, cu_q_lens_host=None,
                         page_writable_host=None) -> None:
    """Host-side checks of an append's tables (numpy arrays or None); raises MvrError."""
    import numpy as np

    keep = []

    def ptr(x, dt=np.int32):
        if x is None:
            return None
        x = np.ascontiguousarray(x, dtype=dt)
        keep.append(x)
        return x.ctypes.data

    _check(load_library().mvr_rope_append_validate(ctypes.byref(args), ptr(block_tables_host), ptr(seq_lens_host),
                                                   ptr(cu_q_lens_host), ptr(page_writable_host, np.uint8)))


def make_cascade_groups(group_cu_q_lens, group_prefix_lens, group_block_tables, seq_prefix_lens, *,
                        max_group_q_len: int, max_prefix_len: int, sum_prefix_lens: int = 0) -> CascadeGroups:
    """Prefix groups for paged_attention_cascade: device int32 tensors (group tensors may be None when there is no
    group); members of a group are consecutive sequences."""
    g = CascadeGroups()
    g.num_groups = 0 if group_prefix_lens is None else int(group_prefix_lens.numel())
    g.max_group_q_len = max_group_q_len
    g.max_prefix_len = max_prefix_len
    g.group_cu_q_lens = group_cu_q_lens.data_ptr() if group_cu_q_lens is not None else None
    g.group_prefix_lens = group_prefix_lens.data_ptr() if group_prefix_lens is not None else None
    g.group_block_tables = group_block_tables.data_ptr() if group_block_tables is not None else None
    g.seq_prefix_lens = seq_prefix_lens.data_ptr()
    g.sum_prefix_lens = int(sum_prefix_lens)
    # Raw device addresses: keep the tables alive with the struct (tables passed as temporaries would
    # otherwise be freed, and their memory reused, e.g. by the call's own output, before the kernels read them).
    g._keep = (group_cu_q_lens, group_prefix_lens, group_block_tables, seq_prefix_lens)
    return g


def paged_attention_cascade(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, groups: CascadeGroups,
                            out=None, *, max_q_len: int, max_seq_len: int, scale: float = 0.0, workspace=None,
                            stream=None, sum_seq_lens: int = 0, seq_lens_host=None, cu_q_lens_host=None):
    """paged_attention with each group's shared prefix attended once; returns out [Hq, total_q, D].  (With the
    sum_prefix_lens hint showing little sharing, the library runs the plain call instead.)"""
    torch = _torch()
    with _stream_scope(stream, q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, workspace,
                       *groups._keep):
        if out is None:
            out = torch.empty_like(q, memory_format=torch.contiguous_format)
        a = make_args(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, out, max_q_len=max_q_len,
                      max_seq_len=max_seq_len, scale=scale, stream=stream, sum_seq_lens=sum_seq_lens,
                      seq_lens_host=seq_lens_host, cu_q_lens_host=cu_q_lens_host)
        lib = load_library()
        need = int(lib.mvr_paged_attention_cascade_workspace_size(ctypes.byref(a), ctypes.byref(groups)))
        if need == 0:
            # An invalid call raises with the reason; a valid one (the plain path, at times) needs no workspace.
            _check(lib.mvr_paged_attention_cascade(ctypes.byref(a), ctypes.byref(groups)))
            return out
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = new_workspace(need, q.device)
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
        _check(lib.mvr_paged_attention_cascade(ctypes.byref(a), ctypes.byref(groups)))
    return out


def validate_cascade(args: PagedAttentionArgs, groups: CascadeGroups, block_tables_host=None, seq_lens_host=None,
                     cu_q_lens_host=None, group_cu_q_lens_host=None, group_prefix_lens_host=None,
                     group_block_tables_host=None, seq_prefix_lens_host=None) -> None:
    """Host-side checks of the prefix groups (numpy int32 arrays or None); raises MvrError."""
    import numpy as np

    keep = []

    def ptr(x):
        if x is None:
            return None
        x = np.ascontiguousarray(x, dtype=np.int32)
        keep.append(x)
        return x.ctypes.data

    _check(load_library().mvr_paged_attention_cascade_validate(
        ctypes.byref(args), ctypes.byref(groups), ptr(block_tables_host), ptr(seq_lens_host), ptr(cu_q_lens_host),
        ptr(group_cu_q_lens_host), ptr(group_prefix_lens_host), ptr(group_block_tables_host),
        ptr(seq_prefix_lens_host)))
