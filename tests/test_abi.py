"""CPU-side checks of the C ABI: the library loads, exports every function
include/mvr_attn.h declares, and its host checks reject bad arguments with
the reference's errors (common.rs:447-454, :776-781) before any launch."""
import ctypes
import os
import re
import subprocess

import pytest

import mvr_attn as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mvr_attn.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mvr_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = M.load_library()
    declared = header_functions()
    assert declared, "no functions parsed from the header"
    assert set(declared) == set(M.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", M.library_path()], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (mvr_[a-z0-9_]+)$", out.stdout, flags=re.M))
    assert set(declared) <= exported
    assert M.load_library().mvr_abi_version() == M.ABI_VERSION == 3


def test_product_library_does_not_link_the_oracle():
    out = subprocess.run(["nm", "-D", M.library_path()], capture_output=True, text=True, check=True).stdout
    assert "oracle_" not in out
    ldd = subprocess.run(["ldd", M.library_path()], capture_output=True, text=True).stdout
    assert "liboracle" not in ldd


def _args(**kw):
    a = M.PagedAttentionArgs()
    a.dtype = M.DTYPE_F16
    a.num_seqs = 2
    a.num_q_heads = 32
    a.num_kv_heads = 8
    a.head_dim = 128
    a.page_size = 16
    a.num_pages = 1024
    a.max_pages_per_seq = 64
    a.max_q_len = 1
    a.max_seq_len = 1024
    fake = 1 << 20  # aligned dummy addresses: these calls never launch
    a.q = a.key_pool = a.value_pool = a.block_tables = a.seq_lens = a.cu_q_lens = a.out = fake
    a.q_stride_head = 2 * 128
    a.q_stride_token = 128
    a.out_stride_head = 2 * 128
    a.out_stride_token = 128
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _call(a):
    lib = M.load_library()
    rc = lib.mvr_paged_attention(ctypes.byref(a))
    return rc, lib.mvr_last_error().decode()


@pytest.mark.parametrize("field,value,code,msg", [
    ("dtype", 7, M.MVR_E_UNSUPPORTED, "dtype"),
    ("num_seqs", 0, M.MVR_E_INVALID_ARGUMENT, "forward requires at least one request"),
    ("num_kv_heads", 5, M.MVR_E_INVALID_ARGUMENT, "not a multiple"),
    ("head_dim", 80, M.MVR_E_UNSUPPORTED, "head_dim"),
    ("page_size", 0, M.MVR_E_INVALID_ARGUMENT, "page_size must be positive"),
    ("max_q_len", 0, M.MVR_E_INVALID_ARGUMENT, "at least one token"),
    ("max_pages_per_seq", 60, M.MVR_E_PAGES_UNCOVERED, "leaving 64 tokens uncovered"),
    ("q", 1 + (1 << 20), M.MVR_E_INVALID_ARGUMENT, "aligned"),
    ("q_stride_token", 100, M.MVR_E_INVALID_ARGUMENT, "aligned"),
    ("seq_lens", None, M.MVR_E_INVALID_ARGUMENT, "required"),
    ("total_q", 1, M.MVR_E_INVALID_ARGUMENT, "total_q 1 is outside"),  # fewer tokens than sequences
    ("total_q", 3, M.MVR_E_INVALID_ARGUMENT, "total_q 3 is outside"),  # more than num_seqs * max_q_len
    ("total_q", -1, M.MVR_E_INVALID_ARGUMENT, "total_q -1 is outside"),
])
def test_scalar_checks_reject_before_launch(field, value, code, msg):
    rc, err = _call(_args(**{field: value}))
    assert rc == code
    assert msg in err


@pytest.mark.parametrize("head_dim", [16, 48, 80, 112, 288, 512])
def test_head_dims_off_the_multiples_of_32_up_to_256_are_refused(head_dim):
    rc, err = _call(_args(head_dim=head_dim, q_stride_head=64 * head_dim, q_stride_token=head_dim,
                          out_stride_head=64 * head_dim, out_stride_token=head_dim))
    assert rc == M.MVR_E_UNSUPPORTED
    assert f"head_dim {head_dim} is not supported" in err


@pytest.mark.parametrize("dtype", [M.DTYPE_F16, M.DTYPE_F32])
@pytest.mark.parametrize("head_dim", [32, 96, 160, 192, 224, 256])
@pytest.mark.parametrize("page_size", [16, 5])
def test_other_head_dims_plan_the_split_kernel_with_its_merge(dtype, head_dim, page_size):
    # Decode, verification and prefill-sized calls of the head dimensions besides 64 and 128 plan on the host
    # (no device: the sizing path) as split contexts merged from partials in the workspace, so it is never
    # empty; page size 5 adds the repack into 16-token pages.
    lib = M.load_library()
    for q_len in (1, 5, 100):
        a = _args(dtype=dtype, head_dim=head_dim, page_size=page_size, max_q_len=q_len, max_seq_len=1024 + q_len,
                  max_pages_per_seq=(1024 + q_len + page_size - 1) // page_size, q_stride_head=64 * q_len * head_dim,
                  q_stride_token=head_dim, out_stride_head=64 * q_len * head_dim, out_stride_token=head_dim)
        size = lib.mvr_paged_attention_workspace_size(ctypes.byref(a))
        assert size > 0, (head_dim, page_size, q_len, lib.mvr_last_error().decode())


def test_errors_are_per_thread_under_concurrent_calls():
    # Several backends (one OS thread each, server/mod.rs:380-391) may call the library at once; each
    # thread must read back its own error.  ctypes drops the GIL around foreign calls, so the
    # threads' checks and error writes overlap in the library.
    import threading
    cases = [("dtype", 7, M.MVR_E_UNSUPPORTED, "dtype"),
             ("num_kv_heads", 5, M.MVR_E_INVALID_ARGUMENT, "not a multiple"),
             ("head_dim", 80, M.MVR_E_UNSUPPORTED, "head_dim"),
             ("max_pages_per_seq", 60, M.MVR_E_PAGES_UNCOVERED, "leaving 64 tokens uncovered"),
             ("q_stride_token", 100, M.MVR_E_INVALID_ARGUMENT, "aligned"),
             ("seq_lens", None, M.MVR_E_INVALID_ARGUMENT, "required"),
             ("max_q_len", 0, M.MVR_E_INVALID_ARGUMENT, "at least one token"),
             ("page_size", 0, M.MVR_E_INVALID_ARGUMENT, "page_size must be positive")]
    start = threading.Barrier(len(cases))
    failures = []

    def worker(field, value, code, msg):
        a = _args(**{field: value})
        start.wait()
        for _ in range(300):
            rc, err = _call(a)
            if rc != code or msg not in err:
                failures.append((field, rc, err))
                return

    threads = [threading.Thread(target=worker, args=c) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not failures, failures[:3]


def test_workspace_too_small_is_rejected():
    a = _args(max_seq_len=1024)
    need = M.workspace_size(a)
    assert need > 0  # 2 sequences x 8 kv heads cannot fill the GPU without splitting the context
    a.workspace = 1 << 20
    a.workspace_bytes = need - 1
    rc, err = _call(a)
    assert rc == M.MVR_E_WORKSPACE and "smaller than" in err


def test_page_sizes_off_16_in_place_or_repacked():
    # Any page size is accepted (the reference's own tests use 2 and 3).  Decode-sized calls read pages of 2 or
    # more tokens in place: the workspace holds only their partials, as with 16-token pages.  Calls that take
    # the chunked-prefill kernel read them in place where each of its 64-lane loads' token rows lie in one page
    # (head_dim 64 and 128, page sizes a multiple of the tokens per load); those calls with other page sizes,
    # and pages of one token, repack each sequence's tokens into 16-token pages in the workspace first, then run
    # the plan of that layout.
    pool = 2 * 64 * 8 * 16 * 128 * 2  # sequences x pages16 x kv heads x 16 tokens x head_dim x f16
    p16 = M.workspace_size(_args(max_seq_len=1024))
    assert M.workspace_size(_args(max_seq_len=1024, page_size=3, max_pages_per_seq=342)) == p16
    assert M.workspace_size(_args(max_seq_len=1024, page_size=40, max_pages_per_seq=26)) == p16
    a1 = _args(max_seq_len=1024, page_size=1, max_pages_per_seq=1024)
    need = M.workspace_size(a1)
    assert need >= 2 * pool + 2 * 64 * 4 + p16
    a1.workspace = 1 << 20
    a1.workspace_bytes = need - 1
    rc, err = _call(a1)
    assert rc == M.MVR_E_WORKSPACE and "smaller than" in err
    prefill16 = M.workspace_size(_args(max_seq_len=1024, max_q_len=256))
    assert M.workspace_size(_args(max_seq_len=1024, max_q_len=256, page_size=3, max_pages_per_seq=342)) >= \
        2 * pool + 2 * 64 * 4 + prefill16
    # In place: F16 D=128 loads cover 4 tokens (multiples of 4), D=64 8, F32 D=128 2, F32 D=64 4.
    in_place = [(M.DTYPE_F16, 128, 4), (M.DTYPE_F16, 128, 8), (M.DTYPE_F16, 128, 12), (M.DTYPE_F16, 64, 8),
                (M.DTYPE_F16, 64, 24), (M.DTYPE_F32, 128, 2), (M.DTYPE_F32, 128, 6), (M.DTYPE_F32, 64, 4)]
    repacked = [(M.DTYPE_F16, 128, 6), (M.DTYPE_F16, 64, 4), (M.DTYPE_F16, 64, 12), (M.DTYPE_F32, 128, 3),
                (M.DTYPE_F32, 64, 2), (M.DTYPE_F16, 96, 8)]
    for dtype, d, ps in in_place + repacked:
        kw = dict(dtype=dtype, head_dim=d, q_stride_head=2 * d, q_stride_token=d, out_stride_head=2 * d,
                  out_stride_token=d, max_seq_len=1024, max_q_len=256)
        base = M.workspace_size(_args(**kw))
        got = M.workspace_size(_args(page_size=ps, max_pages_per_seq=-(-1024 // ps), **kw))
        es = 2 if dtype == M.DTYPE_F16 else 4
        if (dtype, d, ps) in in_place:
            assert got == base, (dtype, d, ps, got, base)
        else:
            assert got >= 2 * (2 * 64 * 8 * 16 * d * es) + base, (dtype, d, ps, got, base)
    # Token pages keep offsets within a page of all KV heads in 32 bits: a decode call on pages of 2^31
    # elements or more (8 KV heads x 2,097,153 tokens x 128) is repacked instead.
    huge = (1 << 21) + 1
    assert M.workspace_size(_args(max_seq_len=1024, page_size=huge - 2, max_pages_per_seq=1)) == p16
    assert M.workspace_size(_args(max_seq_len=1024, page_size=huge, max_pages_per_seq=1)) >= 2 * pool + p16
    # A page size that does not cover max_seq_len is still the reference's error.
    rc, err = _call(_args(max_seq_len=1024, page_size=3, max_pages_per_seq=300))
    assert rc == M.MVR_E_PAGES_UNCOVERED and "leaving 124 tokens uncovered" in err


def test_block_merge_plan_needs_no_workspace():
    # The batch-64 x 8K decode splits every context into one block's worth of partitions (4): they merge in
    # LDS, so the call needs no workspace.  A ragged length hint plans the separate merge again.
    uniform = _args(num_seqs=64, max_seq_len=8192, max_pages_per_seq=512, sum_seq_lens=64 * 8192)
    assert M.workspace_size(uniform) == 0
    ragged = _args(num_seqs=64, max_seq_len=8192, max_pages_per_seq=512, sum_seq_lens=64 * 8192 - 4096)
    assert M.workspace_size(ragged) > 0


def _partial_bytes(units, tile_rows, d):
    """Workspace of a split plan: fp32 partial rows [units * tile_rows][d] and their (m, l), each 256-aligned."""
    rows = units * tile_rows
    up = lambda x: (x + 255) // 256 * 256
    return up(rows * d * 4) + up(rows * 2 * 4)


def _one_token_rows(num_seqs, hq, d, **kw):
    return _args(num_seqs=num_seqs, num_q_heads=hq, head_dim=d, q_stride_head=num_seqs * d, q_stride_token=d,
                 out_stride_head=num_seqs * d, out_stride_token=d, **kw)


def test_long_context_plans_cap_partitions_at_128():
    # One 32K-token sequence over Qwen2-0.5B's 2 KV heads: filling the 2,048 planned slots alone would split its
    # 2,048 chunks down to the 4-chunk floor (512 partitions per KV head); the planner caps a tile at 128.
    a = _one_token_rows(1, 14, 64, num_kv_heads=2, max_seq_len=32768, max_pages_per_seq=2048)
    assert M.workspace_size(a) == _partial_bytes(2 * 128, 16, 64)


def test_large_f16_head_dim_64_calls_plan_three_wavefronts_per_simd():
    # 64 x 16K tokens of F16 K/V at head_dim 64 (537 MB) plan for 1.5x the 2,048 slots: 1,536 units per KV head,
    # 24 partitions per sequence.  A 64 x 4K batch (134 MB, below 256 MiB) keeps the 2,048 slots: 16 partitions,
    # which fit one 16-wavefront block and merge in LDS (no workspace); under the larger target they would not.
    big = _one_token_rows(64, 14, 64, num_kv_heads=2, max_seq_len=16384, max_pages_per_seq=1024, num_pages=65536)
    assert M.workspace_size(big) == _partial_bytes(64 * 2 * 24, 16, 64)
    small = _one_token_rows(64, 14, 64, num_kv_heads=2, max_seq_len=4096, max_pages_per_seq=256, num_pages=16384)
    assert M.workspace_size(small) == 0


def test_validate_mirrors_reference_errors():
    a = _args()
    bt = [[i for i in range(64)], [64 + i for i in range(64)]]
    M.validate(a, bt, [1024, 17], [0, 1, 2])
    with pytest.raises(M.MvrError, match="outside a pool of 1024 pages") as e:
        M.validate(a, [[5000] * 64, bt[1]], [1024, 17], [0, 1, 2])
    assert e.value.code == M.MVR_E_PAGE_ID
    with pytest.raises(M.MvrError, match="reports sequence length 0") as e:
        M.validate(_args(max_q_len=2), bt, [0, 17], [0, 2, 3])
    assert e.value.code == M.MVR_E_LENGTH_MISMATCH
    with pytest.raises(M.MvrError, match="at least one token"):
        M.validate(a, bt, [1024, 17], [0, 0, 1])
    with pytest.raises(M.MvrError, match="max_seq_len"):
        M.validate(a, bt, [2000, 17], [0, 1, 2])
    # q and out hold total_q tokens: the packed count may not exceed it
    with pytest.raises(M.MvrError, match="exceeds total_q = 3"):
        M.validate(_args(max_q_len=2, total_q=3), bt, [1024, 17], [0, 2, 4])
    M.validate(_args(max_q_len=2, total_q=4), bt, [1024, 17], [0, 2, 4])
    with pytest.raises(M.MvrError, match="smaller than max_q_len"):
        M.validate(_args(num_seqs=1, max_q_len=5, total_q=4, cu_q_lens=None), bt, [1024], None)


def _mixed_args(q_lens, seq_lens, hints, **kw):
    """Scalar-only args (never launched) of a Llama-3-8B-shaped F16 call with these requests."""
    import numpy as np
    q_lens, seq_lens = np.asarray(q_lens, np.int32), np.asarray(seq_lens, np.int32)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    kw.setdefault("total_q", int(cu[-1]))
    a = _args(num_seqs=len(q_lens), max_q_len=int(q_lens.max()), max_seq_len=int(seq_lens.max()),
              max_pages_per_seq=int(seq_lens.max() + 15) // 16, num_pages=1 << 16, sum_seq_lens=int(seq_lens.sum()),
              **kw)
    if hints:
        a.seq_lens_host = seq_lens.ctypes.data
        a.cu_q_lens_host = cu.ctypes.data
    a._keep = (seq_lens, cu)
    return a


def test_mixed_batch_without_host_tables_plans_like_the_hinted_call():
    # A scheduler step (decodes first, then the prefill chunks, scheduler.rs:258-271) without host copies of the
    # length tables: total_q says how many prefill-sized requests the tail holds, so the plans (and the
    # workspace they need) match the hinted call's.
    step = dict(q_lens=[1] * 63 + [256], seq_lens=[8192] * 63 + [2304])
    assert M.workspace_size(_mixed_args(**step, hints=False)) == M.workspace_size(_mixed_args(**step, hints=True))
    two = dict(q_lens=[1] * 30 + [200, 200], seq_lens=[4096] * 30 + [1000, 3000])
    assert M.workspace_size(_mixed_args(**two, hints=False)) == M.workspace_size(_mixed_args(**two, hints=True))
    # A call whose tokens could fill every sequence with a prefill chunk runs as one prefill launch, as with
    # hints that show one class; with total_q unknown it keeps the two launches (launch 0 over the decode
    # shape: its own partial slots).
    chunks = dict(q_lens=[256] * 4, seq_lens=[2304] * 4)
    one = M.workspace_size(_mixed_args(**chunks, hints=True))
    assert M.workspace_size(_mixed_args(**chunks, hints=False)) == one
    assert M.workspace_size(_mixed_args(**chunks, hints=False, total_q=0)) != one


def test_request_level_entry_checks_lengths():
    lib = M.load_library()
    dims = M.AttentionDimensions(14, 2, 64, 511, 1)
    lay = M.PagedCacheLayoutC(1 << 20, 1 << 20, 64, 1 << 20, 32, 16, 513)
    rc = lib.mvr_forward_paged_attention(M.DTYPE_F32, ctypes.byref(dims), ctypes.byref(lay), 1 << 20, 1 << 20, None, 0,
                                         None)
    assert rc == M.MVR_E_LENGTH_MISMATCH
    assert "paged KV cache reports sequence length 513, expected 512" in lib.mvr_last_error().decode()
    lay = M.PagedCacheLayoutC(1 << 20, 1 << 20, 64, 1 << 20, 31, 16, 512)
    rc = lib.mvr_forward_paged_attention(M.DTYPE_F32, ctypes.byref(dims), ctypes.byref(lay), 1 << 20, 1 << 20, None, 0,
                                         None)
    assert rc == M.MVR_E_PAGES_UNCOVERED
    assert "leaving 16 tokens uncovered" in lib.mvr_last_error().decode()


def test_reconstruct_contiguous_rejects_like_the_reference():
    lib = M.load_library()
    rc = lib.mvr_reconstruct_contiguous(M.DTYPE_F16, 1 << 20, 8, 2, 16, 64, 1 << 20, 0, 0, 1 << 20, None)
    assert rc == M.MVR_E_INVALID_ARGUMENT
    assert "cannot reconstruct an empty KV cache" in lib.mvr_last_error().decode()  # paged_cache.rs:383-385
    rc = lib.mvr_reconstruct_contiguous(M.DTYPE_F16, 1 << 20, 8, 2, 16, 64, 1 << 20, 2, 40, 1 << 20, None)
    assert rc == M.MVR_E_PAGES_UNCOVERED and "leaving 8 tokens uncovered" in lib.mvr_last_error().decode()
    rc = lib.mvr_reconstruct_contiguous(5, 1 << 20, 8, 2, 16, 64, 1 << 20, 2, 20, 1 << 20, None)
    assert rc == M.MVR_E_UNSUPPORTED


def _rope_args(**kw):
    a = M.RopeAppendArgs()
    a.dtype = M.DTYPE_F16
    a.rope_type = M.ROPE_NEOX
    a.num_seqs = 2
    a.num_q_heads = 8
    a.num_kv_heads = 2
    a.head_dim = 64
    a.page_size = 4
    a.num_pages = 16
    a.max_pages_per_seq = 4
    a.total_q = 5
    a.max_seq_len = 16
    a.rope_len = 32
    fake = 1 << 20  # aligned dummy addresses: these calls never launch
    a.q = a.k = a.v = a.cos_table = a.sin_table = a.block_tables = a.seq_lens = a.cu_q_lens = fake
    a.q_out = a.key_pool = a.value_pool = fake
    a.q_stride_head = a.q_out_stride_head = 5 * 64
    a.k_stride_head = a.v_stride_head = 5 * 64
    a.q_stride_token = a.q_out_stride_token = a.k_stride_token = a.v_stride_token = 64
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code,msg", [
    ("rope_type", 2, M.MVR_E_UNSUPPORTED, "rope_type"),
    ("head_dim", 60, M.MVR_E_UNSUPPORTED, "head_dim"),
    ("total_q", 0, M.MVR_E_INVALID_ARGUMENT, "cannot append an empty KV-cache tensor"),
    ("rope_len", 15, M.MVR_E_INVALID_ARGUMENT, "rotary tables hold 15 positions"),
    ("max_pages_per_seq", 3, M.MVR_E_PAGES_UNCOVERED, "cannot hold 16 tokens"),
    ("k", 4 + (1 << 20), M.MVR_E_INVALID_ARGUMENT, "aligned"),
    ("v_stride_token", 66, M.MVR_E_INVALID_ARGUMENT, "multiples of 4"),
    ("cu_q_lens", None, M.MVR_E_INVALID_ARGUMENT, "required"),
])
def test_rope_append_scalar_checks_reject_before_launch(field, value, code, msg):
    lib = M.load_library()
    rc = lib.mvr_rope_append(ctypes.byref(_rope_args(**{field: value})))
    assert rc == code
    assert msg in lib.mvr_last_error().decode()


def test_rope_append_validate_mirrors_reference_errors():
    a = _rope_args()
    bt = [[3, 7, 1, 0], [9, 2, 0, 0]]
    writable = [1] * 16
    M.validate_rope_append(a, bt, [10, 6], [0, 3, 5], writable)  # positions 7..9 and 4..5
    with pytest.raises(M.MvrError, match="cannot append an empty KV-cache tensor"):
        M.validate_rope_append(a, bt, [10, 6], [0, 5, 5])
    w = list(writable)
    w[1] = 0  # page 1 holds positions 8..9 of request 0: written and shared
    with pytest.raises(M.MvrError, match="cannot mutate written physical page 1") as e:
        M.validate_rope_append(a, bt, [10, 6], [0, 3, 5], w)
    assert e.value.code == M.MVR_E_READ_ONLY_PAGE
    w = list(writable)
    w[3] = 0  # page 3 holds positions 0..3: not written by this append
    M.validate_rope_append(a, bt, [10, 6], [0, 3, 5], w)
    with pytest.raises(M.MvrError, match="written by more than one request"):
        M.validate_rope_append(a, [[3, 7, 2, 0], [9, 2, 0, 0]], [10, 6], [0, 3, 5])
    with pytest.raises(M.MvrError, match="outside a pool of 16 pages") as e:
        M.validate_rope_append(a, [[3, 7, 99, 0], [9, 2, 0, 0]], [10, 6], [0, 3, 5])
    assert e.value.code == M.MVR_E_PAGE_ID
    with pytest.raises(M.MvrError, match="after appending"):
        M.validate_rope_append(a, bt, [2, 6], [0, 3, 5])
    with pytest.raises(M.MvrError, match="total_q"):
        M.validate_rope_append(a, bt, [10, 6], [0, 3, 4])


def test_argument_structs_keep_their_tensors_alive():
    # The structs carry raw addresses.  Tables passed as temporaries must live as long as the struct: freed,
    # their memory can be reused (by the call's own output, say) before the kernels read them.
    import gc
    import weakref

    torch = pytest.importorskip("torch")
    refs = []

    def tmp(*shape, dtype=torch.int32):
        t = torch.zeros(*shape, dtype=dtype)
        refs.append(weakref.ref(t))
        return t

    class NullStream:  # no launch happens here: any handle will do
        cuda_stream = 0

    g = M.make_cascade_groups(tmp(3), tmp(2), tmp(2, 4), tmp(4), max_group_q_len=2, max_prefix_len=32)
    a = M.make_args(tmp(8, 4, 64, dtype=torch.float16), tmp(16, 1, 2, 16, 64, dtype=torch.float16),
                    tmp(16, 1, 2, 16, 64, dtype=torch.float16), tmp(4, 4), tmp(4), tmp(5),
                    tmp(8, 4, 64, dtype=torch.float16), max_q_len=1, max_seq_len=64, stream=NullStream())
    r = M.make_rope_append_args(tmp(8, 4, 64, dtype=torch.float16), tmp(2, 4, 64, dtype=torch.float16),
                                tmp(2, 4, 64, dtype=torch.float16), tmp(64, 32, dtype=torch.float16),
                                tmp(64, 32, dtype=torch.float16), tmp(4, 4), tmp(4), tmp(5),
                                tmp(16, 1, 2, 16, 64, dtype=torch.float16), tmp(16, 1, 2, 16, 64, dtype=torch.float16),
                                tmp(8, 4, 64, dtype=torch.float16), max_seq_len=64, stream=NullStream())
    gc.collect()
    assert all(w() is not None for w in refs), "a tensor behind a struct address was freed"
    assert g.seq_prefix_lens == g._keep[3].data_ptr() and a.cu_q_lens == a._keep[5].data_ptr()
    del g, a, r
    gc.collect()
    assert all(w() is None for w in refs)


def _groups(**kw):
    g = M.CascadeGroups()
    g.num_groups = 1
    g.max_group_q_len = 2
    g.max_prefix_len = 32
    fake = 1 << 20
    g.group_cu_q_lens = g.group_prefix_lens = g.group_block_tables = g.seq_prefix_lens = fake
    for k, v in kw.items():
        setattr(g, k, v)
    return g


def test_cascade_scalar_checks_reject_before_launch():
    lib = M.load_library()
    a = _args()
    for kw, msg in [(dict(seq_prefix_lens=None), "seq_prefix_lens is required"),
                    (dict(max_prefix_len=4096), "exceeds max_seq_len"),
                    (dict(num_groups=3), "num_groups 3"),
                    (dict(group_block_tables=None), "group tables are required")]:
        rc = lib.mvr_paged_attention_cascade(ctypes.byref(a), ctypes.byref(_groups(**kw)))
        assert rc == M.MVR_E_INVALID_ARGUMENT, kw
        assert msg in lib.mvr_last_error().decode(), (kw, lib.mvr_last_error())
    assert lib.mvr_paged_attention_cascade_workspace_size(ctypes.byref(a), ctypes.byref(_groups())) > 0


def test_cascade_falls_back_to_the_plain_call_when_sharing_is_small():
    lib = M.load_library()
    size = lambda a, g: lib.mvr_paged_attention_cascade_workspace_size(ctypes.byref(a), ctypes.byref(g))
    # 16 sequences of 5 query tokens, 139264 cached tokens in all; 4 groups share 1024 tokens each: 12288 reads
    # saved (9%), so the call runs as mvr_paged_attention and needs its workspace
    a = _args(num_seqs=16, max_q_len=5, max_seq_len=16384, max_pages_per_seq=1024, num_pages=32768,
              sum_seq_lens=139264)
    small = _groups(num_groups=4, max_group_q_len=20, max_prefix_len=1024, sum_prefix_lens=16 * 1024)
    assert size(a, small) == lib.mvr_paged_attention_workspace_size(ctypes.byref(a))
    state = a.num_q_heads * a.num_seqs * a.max_q_len * a.head_dim * 4  # the cascade's per-row prefix state
    small.sum_prefix_lens = 0  # without the hint the cascade runs as asked
    assert size(a, small) >= state
    # 64 decode sequences behind one 8192-token prompt: 63 * 8192 of 64 * 9344 reads saved (86%)
    b = _args(num_seqs=64, max_q_len=1, max_seq_len=10240, max_pages_per_seq=640, num_pages=40000,
              sum_seq_lens=64 * 9344)
    big = _groups(num_groups=1, max_group_q_len=64, max_prefix_len=8192, sum_prefix_lens=64 * 8192)
    assert size(b, big) >= b.num_q_heads * b.num_seqs * b.head_dim * 4
    assert size(b, big) != lib.mvr_paged_attention_workspace_size(ctypes.byref(b))


def test_cascade_validate_checks_the_groups():
    # two sequences of one token each, 16-token pages; both share the first 32 tokens (2 pages)
    a = _args(max_q_len=1, max_seq_len=1024)
    bt = [[7, 9] + list(range(20, 82)), [7, 9] + list(range(100, 162))]
    seq_lens, cu = [200, 300], [0, 1, 2]
    gbt = [bt[0]]
    ok = dict(group_cu_q_lens_host=[0, 2], group_prefix_lens_host=[32], group_block_tables_host=gbt,
              seq_prefix_lens_host=[32, 32])
    M.validate_cascade(a, _groups(), bt, seq_lens, cu, **ok)
    bad = [(dict(group_prefix_lens_host=[24]), "not a multiple of page_size"),
           (dict(group_cu_q_lens_host=[1, 2]), "sequence 0 is in no group"),
           (dict(seq_prefix_lens_host=[32, 16]), "its group's prefix is 32"),
           (dict(group_block_tables_host=[[7, 8] + bt[0][2:]]), "differs from its group's shared page")]
    for change, msg in bad:
        kw = dict(ok)
        kw.update(change)
        with pytest.raises(M.MvrError, match=msg):
            M.validate_cascade(a, _groups(), bt, seq_lens, cu, **kw)
    with pytest.raises(M.MvrError, match="exceeds sequence 0's 0 cached tokens"):
        M.validate_cascade(a, _groups(), bt, [1, 300], cu, **ok)
    with pytest.raises(M.MvrError, match="is in no group"):
        M.validate_cascade(a, _groups(num_groups=0), bt, seq_lens, cu, group_cu_q_lens_host=[0],
                           seq_prefix_lens_host=[0, 32])
    # a group must begin and end on sequence boundaries (sequence 0 holds packed tokens 0 and 1)
    a2 = _args(max_q_len=2, max_seq_len=1024)
    with pytest.raises(M.MvrError, match="does not start at a sequence boundary"):
        M.validate_cascade(a2, _groups(), bt, seq_lens, [0, 2, 3], group_cu_q_lens_host=[1, 3],
                           group_prefix_lens_host=[32], group_block_tables_host=gbt, seq_prefix_lens_host=[0, 32])


def test_workloads_match_stated_sizes():
    import workloads as W

    w3 = W.llama3_8b_decode_b64_8k_f16()
    assert w3.algorithmic_bytes() == 2_148_663_296
    assert w3.kv_bytes() == 2_147_483_648
    w4 = W.qwen2_7b_chunked_prefill_f16()
    assert w4.flops() == 31_951_159_296
    assert w4.kv_bytes() + 2 * 28 * 1024 * 128 * 2 == 33_554_432
    w1 = W.qwen2_05b_decode_f32()
    assert w1.kv_bytes() == 524_288
    w5 = W.llama3_8b_spec_verify_f16()
    assert w5.kv_bytes() - w5.unique_kv_bytes() == 50_331_648
    # shared prefixes: 4 groups, identical physical ids inside a group, disjoint elsewhere
    bt = w5.block_tables
    for s in range(16):
        assert (bt[s, :64] == bt[(s // 4) * 4, :64]).all()
    used = set()
    for s in range(16):
        n = -(-int(w5.seq_lens[s]) // 16)
        ids = bt[s, 64 if s % 4 else 0:n].tolist()
        assert not used.intersection(ids)
        used.update(ids)
    assert len(used) == w5.num_pages


def test_noalloc_refuses_calls_larger_than_its_scratch():
    """One-token pages repack the batch's K/V into the scratch: 64 sequences of 8K tokens need ~2 GiB, more
    than the static scratch holds, so the call returns MVR_E_WORKSPACE before launching anything (or touching a
    device: the refusal needs none, and the dummy addresses are never read)."""
    lib = M.load_library()
    a = M.PagedAttentionArgs()
    a.dtype, a.num_seqs, a.num_q_heads, a.num_kv_heads, a.head_dim = M.DTYPE_F16, 64, 32, 8, 128
    a.page_size, a.num_pages, a.max_pages_per_seq, a.max_q_len, a.max_seq_len = 1, 1 << 20, 8192, 1, 8192
    fake = 1 << 20
    a.q = a.key_pool = a.value_pool = a.block_tables = a.seq_lens = a.cu_q_lens = a.out = fake
    a.q_stride_head, a.q_stride_token, a.out_stride_head, a.out_stride_token = 64 * 128, 128, 64 * 128, 128
    assert M.workspace_size(a) > M.NOALLOC_SCRATCH_BYTES
    rc = lib.mvr_paged_attention_noalloc(ctypes.byref(a))
    assert rc == M.MVR_E_WORKSPACE
    assert "static scratch" in lib.mvr_last_error().decode()
