"""ORACLE — test infrastructure only.

ctypes binding for liboracle.so, the CPU restatement of mini-vllm-rs page-wise
attention (src/models/backends/common.rs:739-978) and of the RoPE + KV append
that precedes it (common.rs:294-320, :344-359; kv_cache/paged_cache.rs:290-327;
kv_cache/physical_page_pool.rs:188-209).  Imported only by the test suite, the
smoke check and the benchmark's CPU-baseline leg.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16 = 0, 1
REF_CONCAT_V, REF_PAGEWISE_V, EXACT_F64 = 0, 1, 2

E_INVALID, E_LENGTH, E_UNCOVERED, E_PAGE_ID, E_NO_PAGES, E_ALLOC = -1, -2, -3, -4, -5, -6

ROPE_NEOX, ROPE_INTERLEAVED = 0, 1
(APPEND_E_INVALID, APPEND_E_EMPTY, APPEND_E_MISSING, APPEND_E_PAGE_ID, APPEND_E_READ_ONLY,
 APPEND_E_ROPE_RANGE) = -1, -2, -3, -4, -5, -6


class OracleDims(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int),
        ("num_q_heads", ctypes.c_int),
        ("num_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("cached_kv_len", ctypes.c_int),
        ("q_len", ctypes.c_int),
    ]


class OracleBatch(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int),
        ("num_seqs", ctypes.c_int),
        ("num_q_heads", ctypes.c_int),
        ("num_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("page_size", ctypes.c_int),
        ("num_pages", ctypes.c_int64),
        ("max_pages_per_seq", ctypes.c_int),
        ("q", ctypes.c_void_p),
        ("q_stride_head", ctypes.c_int64),
        ("q_stride_token", ctypes.c_int64),
        ("key_pool", ctypes.c_void_p),
        ("value_pool", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("cu_q_lens", ctypes.c_void_p),
    ]


class OracleRopeAppendBatch(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int),
        ("rope_type", ctypes.c_int),
        ("num_seqs", ctypes.c_int),
        ("num_q_heads", ctypes.c_int),
        ("num_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("page_size", ctypes.c_int),
        ("num_pages", ctypes.c_int64),
        ("max_pages_per_seq", ctypes.c_int),
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
        ("rope_len", ctypes.c_int),
        ("block_tables", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("cu_q_lens", ctypes.c_void_p),
        ("q_out", ctypes.c_void_p),
        ("q_out_stride_head", ctypes.c_int64),
        ("q_out_stride_token", ctypes.c_int64),
        ("key_pool", ctypes.c_void_p),
        ("value_pool", ctypes.c_void_p),
    ]


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_forward_paged_attention.restype = ctypes.c_int
        L.oracle_forward_paged_attention.argtypes = [
            ctypes.POINTER(OracleDims), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_char_p, ctypes.c_size_t,
        ]
        L.oracle_forward_contiguous_attention.restype = ctypes.c_int
        L.oracle_forward_contiguous_attention.argtypes = [
            ctypes.POINTER(OracleDims), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
            ctypes.c_int, ctypes.c_void_p,
        ]
        L.oracle_reconstruct_contiguous.restype = ctypes.c_int
        L.oracle_reconstruct_contiguous.argtypes = [
            ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
        ]
        L.oracle_paged_attention.restype = ctypes.c_int
        L.oracle_paged_attention.argtypes = [ctypes.POINTER(OracleBatch), ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        L.oracle_num_threads.restype = ctypes.c_int
        L.oracle_rope.restype = ctypes.c_int
        L.oracle_rope.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_void_p]
        L.oracle_rope_f64.restype = ctypes.c_int
        L.oracle_rope_f64.argtypes = L.oracle_rope.argtypes[1:]
        L.oracle_append_pages.restype = ctypes.c_int
        L.oracle_append_pages.argtypes = [
            ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
        ]
        L.oracle_rope_append.restype = ctypes.c_int
        L.oracle_rope_append.argtypes = [ctypes.POINTER(OracleRopeAppendBatch), ctypes.c_char_p, ctypes.c_size_t]
        _lib = L
    return _lib


def _np_dtype(dtype: int):
    return np.float16 if dtype == F16 else np.float32


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class OracleError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message or f"oracle error {code}")
        self.code = code


def forward_paged_attention(request_q, key_pool, value_pool, page_ids, per_page_token_count, cached_token_count,
                            num_q_heads, num_kv_heads, head_dim, cached_kv_len, q_len, dtype=F32,
                            mode=REF_CONCAT_V):
    """Request-level oracle: request_q [1,Hq,q,D], pools [N,1,Hkv,P,D]; returns [Hq,q,D] float64."""
    npd = _np_dtype(dtype)
    q = np.ascontiguousarray(request_q, dtype=npd)
    kp = np.ascontiguousarray(key_pool, dtype=npd)
    vp = np.ascontiguousarray(value_pool, dtype=npd)
    ids = np.ascontiguousarray(page_ids, dtype=np.int64)
    out = np.zeros((num_q_heads, q_len, head_dim), dtype=np.float64)
    dims = OracleDims(dtype, num_q_heads, num_kv_heads, head_dim, cached_kv_len, q_len)
    err = ctypes.create_string_buffer(256)
    rc = lib().oracle_forward_paged_attention(
        ctypes.byref(dims), _ptr(q), _ptr(kp), _ptr(vp), kp.shape[0], _ptr(ids) if ids.size else None, ids.size,
        per_page_token_count, cached_token_count, mode, _ptr(out), err, 256)
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    return out


def forward_contiguous_attention(request_q, full_k, full_v, num_q_heads, num_kv_heads, head_dim, cached_kv_len,
                                 q_len, dtype=F32, mode=REF_CONCAT_V):
    npd = _np_dtype(dtype)
    q = np.ascontiguousarray(request_q, dtype=npd)
    k = np.ascontiguousarray(full_k, dtype=npd)
    v = np.ascontiguousarray(full_v, dtype=npd)
    kv_len = k.shape[2]
    out = np.zeros((num_q_heads, q_len, head_dim), dtype=np.float64)
    dims = OracleDims(dtype, num_q_heads, num_kv_heads, head_dim, cached_kv_len, q_len)
    rc = lib().oracle_forward_contiguous_attention(ctypes.byref(dims), _ptr(q), _ptr(k), _ptr(v), kv_len, mode,
                                                   _ptr(out))
    if rc != 0:
        raise OracleError(rc, "")
    return out


def reconstruct_contiguous(pool, page_ids, cached_token_count, dtype=F16):
    npd = _np_dtype(dtype)
    p = np.ascontiguousarray(pool, dtype=npd)
    n, _, hkv, page_size, d = p.shape
    ids = np.ascontiguousarray(page_ids, dtype=np.int64)
    out = np.zeros((hkv, cached_token_count, d), dtype=npd)
    rc = lib().oracle_reconstruct_contiguous(dtype, _ptr(p), hkv, page_size, d, n, _ptr(ids), ids.size,
                                             cached_token_count, _ptr(out))
    if rc != 0:
        raise OracleError(rc, "")
    return out


def paged_attention(q, key_pool, value_pool, block_tables, seq_lens, cu_q_lens, num_q_heads, num_kv_heads,
                    head_dim, page_size, dtype=F16, mode=REF_CONCAT_V, num_threads=0):
    """Batched oracle over the library layout; q [Hq, total_q, D]; returns [Hq, total_q, D] float64."""
    npd = _np_dtype(dtype)
    q = np.ascontiguousarray(q, dtype=npd)
    kp = np.ascontiguousarray(key_pool, dtype=npd)
    vp = np.ascontiguousarray(value_pool, dtype=npd)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    cu = np.ascontiguousarray(cu_q_lens, dtype=np.int32)
    total_q = int(cu[-1])
    assert q.shape == (num_q_heads, total_q, head_dim), q.shape
    out = np.zeros((num_q_heads, total_q, head_dim), dtype=np.float64)
    b = OracleBatch(dtype, len(sl), num_q_heads, num_kv_heads, head_dim, page_size, kp.shape[0], bt.shape[1],
                    _ptr(q), total_q * head_dim, head_dim, _ptr(kp), _ptr(vp), _ptr(bt), _ptr(sl), _ptr(cu))
    rc = lib().oracle_paged_attention(ctypes.byref(b), mode, num_threads, _ptr(out))
    if rc != 0:
        raise OracleError(rc, "batched oracle rejected its input")
    return out


def f32_to_f16_bits(x: float) -> int:
    return lib().oracle_f32_to_f16(x)


def f16_bits_to_f32(h: int) -> float:
    return lib().oracle_f16_to_f32(h)


def rope(x, cos_table, sin_table, start_pos, rope_type=ROPE_NEOX, dtype=F32):
    """forward_rope for one request: x [heads, q_len, D] in dtype; returns the rotated copy."""
    npd = _np_dtype(dtype)
    xa = np.ascontiguousarray(x, dtype=npd)
    c = np.ascontiguousarray(cos_table, dtype=npd)
    s = np.ascontiguousarray(sin_table, dtype=npd)
    heads, q_len, d = xa.shape
    y = np.empty_like(xa)
    rc = lib().oracle_rope(dtype, rope_type, _ptr(xa), heads, q_len, d, _ptr(c), _ptr(s), c.shape[0], start_pos,
                           _ptr(y))
    if rc != 0:
        raise OracleError(rc, "rope rejected its input")
    return y


def rope_f64(x, cos_table, sin_table, start_pos, rope_type=ROPE_NEOX):
    xa = np.ascontiguousarray(x, dtype=np.float64)
    c = np.ascontiguousarray(cos_table, dtype=np.float64)
    s = np.ascontiguousarray(sin_table, dtype=np.float64)
    heads, q_len, d = xa.shape
    y = np.empty_like(xa)
    rc = lib().oracle_rope_f64(rope_type, _ptr(xa), heads, q_len, d, _ptr(c), _ptr(s), c.shape[0], start_pos, _ptr(y))
    if rc != 0:
        raise OracleError(rc, "rope rejected its input")
    return y


def append_pages(key_pool, value_pool, page_ids, cached_token_count, key, value, page_writable=None):
    """append_to_pages into numpy pools [N,1,Hkv,P,D] (modified in place); key/value [Hkv, n, D], any dtype."""
    assert key_pool.flags.c_contiguous and value_pool.flags.c_contiguous
    assert key_pool.dtype == key.dtype == value.dtype == value_pool.dtype
    n_pages, _, hkv, page_size, d = key_pool.shape
    k = np.ascontiguousarray(key)
    v = np.ascontiguousarray(value)
    ids = np.ascontiguousarray(page_ids, dtype=np.int64)
    w = None if page_writable is None else np.ascontiguousarray(page_writable, dtype=np.uint8)
    err = ctypes.create_string_buffer(256)
    rc = lib().oracle_append_pages(key_pool.dtype.itemsize, _ptr(key_pool), _ptr(value_pool), n_pages, hkv,
                                   page_size, d, _ptr(ids) if ids.size else None, ids.size, cached_token_count,
                                   _ptr(k), _ptr(v), k.shape[1], None if w is None else _ptr(w), err, 256)
    if rc != 0:
        raise OracleError(rc, err.value.decode())


def rope_append(q, k, v, cos_table, sin_table, block_tables, seq_lens, cu_q_lens, key_pool, value_pool,
                rope_type=ROPE_NEOX, dtype=F16):
    """Batched RoPE + append over the library layout: q [Hq, total_q, D], k/v [Hkv, total_q, D].
    Returns the rotated q; key_pool / value_pool (numpy) are written in place."""
    npd = _np_dtype(dtype)
    qa = np.ascontiguousarray(q, dtype=npd)
    ka = np.ascontiguousarray(k, dtype=npd)
    va = np.ascontiguousarray(v, dtype=npd)
    c = np.ascontiguousarray(cos_table, dtype=npd)
    s = np.ascontiguousarray(sin_table, dtype=npd)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    cu = np.ascontiguousarray(cu_q_lens, dtype=np.int32)
    assert key_pool.dtype == npd and value_pool.dtype == npd
    assert key_pool.flags.c_contiguous and value_pool.flags.c_contiguous
    hq, total_q, d = qa.shape
    hkv = ka.shape[0]
    q_out = np.empty_like(qa)
    b = OracleRopeAppendBatch(dtype, rope_type, len(sl), hq, hkv, d, key_pool.shape[3], key_pool.shape[0],
                              bt.shape[1], _ptr(qa), total_q * d, d, _ptr(ka), total_q * d, d, _ptr(va),
                              total_q * d, d, _ptr(c), _ptr(s), c.shape[0], _ptr(bt), _ptr(sl), _ptr(cu),
                              _ptr(q_out), total_q * d, d, _ptr(key_pool), _ptr(value_pool))
    err = ctypes.create_string_buffer(256)
    rc = lib().oracle_rope_append(ctypes.byref(b), err, 256)
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    return q_out
