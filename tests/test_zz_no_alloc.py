"""mvr_paged_attention_noalloc (the allocation-free variant of mvr_paged_attention) through the C ABI.

Its output must equal mvr_paged_attention's with a caller workspace bit for bit (same plan, same kernels; only the
scratch memory differs) on consecutive calls that reuse the library's static scratch, the second with a smaller
input; calls needing more scratch than the library holds are refused before any launch; repeated calls change
the device's free memory by nothing.
"""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mvr_attn as M  # noqa: E402
import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()


def _both(w, t, hints=False):
    """(noalloc output, workspace output) for one workload, each into its own NaN-filled output."""
    kw = dict(seq_lens_host=w.seq_lens, cu_q_lens_host=w.cu_q_lens) if hints else {}
    lib = M.load_library()
    out_n = torch.full_like(t["q"], float("nan"))
    a = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out_n,
                    max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()), **kw)
    need = M.workspace_size(a)
    assert need <= M.NOALLOC_SCRATCH_BYTES
    rc = lib.mvr_paged_attention_noalloc(ctypes.byref(a))
    assert rc == 0, lib.mvr_last_error().decode()
    ref = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                            max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()),
                            **kw)
    torch.cuda.synchronize()
    return out_n, ref, need


def test_noalloc_equals_workspace_call_on_consecutive_calls():
    # The verify workload needs the most scratch of the benchmark workloads (about 51 MiB of partials); the
    # Qwen2-0.5B batch after it needs about 3 MiB and runs on what the first call left in the scratch.
    big, small = W.llama3_8b_spec_verify_f16(), W.qwen2_05b_batched_decode_f16()
    tb, ts = W.device_tensors(big, None, seed=1), W.device_tensors(small, None, seed=2)
    n1, r1, need1 = _both(big, tb)
    n2, r2, need2 = _both(small, ts)
    print(f"scratch used: {need1} then {need2} bytes", flush=True)
    assert need1 > need2 > 0
    assert torch.equal(n1, r1)
    assert torch.equal(n2, r2)
    # and back to the large call, then the small one again
    n3, r3, _ = _both(big, tb)
    n4, r4, _ = _both(small, ts)
    assert torch.equal(n3, r1) and torch.equal(n4, r2)


def _long_prefill(dtype):
    """One 130-token chunk on 4,000 cached tokens, 32/8 heads, D=128: 40 row tiles for 256 CUs, so the prefill
    kernel splits the keys and merges the splits from fp32 partials in the scratch."""
    rng = np.random.default_rng(9)
    lens, qlens = np.array([4130], np.int32), np.array([130], np.int32)
    n = -(-4130 // 16)
    bt = rng.permutation(n + 3)[:n].astype(np.int32).reshape(1, n)
    return W.Workload(f"prefill key splits {dtype}", dtype, 32, 8, 128, 16, n + 3, 0.3, lens, qlens, bt, 9)


@pytest.mark.parametrize("case", ["page-size-5-in-place", "repacked-page-size-5", "head-dim-96-repacked",
                                  "mixed-with-hints", "block-merge", "prefill", "prefill-f32", "prefill-key-splits-f16",
                                  "prefill-key-splits-f32", "prefill-token-pages-8"])
def test_noalloc_equals_workspace_call_on_every_plan(case):
    if case in ("page-size-5-in-place", "repacked-page-size-5", "head-dim-96-repacked"):
        # decode and verify rows read 5-token pages in place; with a 100-token chunk the call is prefill-sized
        # and repacks them into 16-token pages in the scratch first (head_dim 96: always repacked, then the
        # split-context kernel's partials in the scratch too)
        hq, hkv, d, P = 32, 8, 96 if case == "head-dim-96-repacked" else 128, 5
        lens = np.array([700, 97, 1500], np.int32)
        qlens = np.array([1, 5, 1] if case == "page-size-5-in-place" else [1, 5, 100], np.int32)
        need = [-(-int(L) // P) for L in lens]
        bt = np.zeros((3, max(need)), np.int32)
        perm = np.random.default_rng(4).permutation(sum(need) + 2).astype(np.int32)
        used = 0
        for s, n in enumerate(need):
            bt[s, :n] = perm[used:used + n]
            used += n
        w = W.Workload("page size 5", "f16", hq, hkv, d, P, sum(need) + 2, 0.3, lens, qlens, bt, 3)
        t = W.device_tensors(w, None, seed=3)
    elif case == "mixed-with-hints":
        w = W.llama3_8b_mixed_decode_prefill_f16(num_decode=15, decode_ctx=4096)
        t = W.device_tensors(w, None, seed=5)
    elif case == "block-merge":
        w = W.llama3_8b_decode_b64_8k_f16()
        t = W.device_tensors(w, None, seed=6)
    elif case.startswith("prefill-key-splits"):
        w = _long_prefill(case.rsplit("-", 1)[1])
        t = W.device_tensors(w, None, seed=9)
    elif case == "prefill-token-pages-8":
        # the prefill kernel reads 8-token pages in place: no repack in the scratch
        w = W.repaged(W.qwen2_7b_chunked_prefill_f16(), 8)
        t = W.device_tensors(w, None, seed=10)
    else:
        w = W.qwen2_7b_chunked_prefill_f16("f32" if case == "prefill-f32" else "f16")
        t = W.device_tensors(w, None, seed=7)
    n, r, need = _both(w, t, hints=(case == "mixed-with-hints"))
    print(f"{case}: scratch {need} bytes", flush=True)
    if case.startswith("prefill-key-splits"):
        assert need > 0  # the split partials live in the scratch
    assert torch.equal(n, r)


def test_noalloc_calls_leave_free_device_memory_unchanged():
    w = W.llama3_8b_spec_verify_f16()
    t = W.device_tensors(w, None, seed=8)
    out = torch.empty_like(t["q"])
    kw = dict(max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    M.paged_attention_noalloc(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                              t["cu_q_lens"], out, **kw)  # first use on this device: the scratch's module is loaded
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    alloc0 = torch.cuda.memory_allocated()
    for _ in range(5):
        M.paged_attention_noalloc(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                                  t["cu_q_lens"], out, **kw)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.cuda.memory_allocated() == alloc0
