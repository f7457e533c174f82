"""The attention entry points captured in a HIP graph: every plan's launches (split-context kernel and merge, block
merge, 32-row verify tiles, chunked prefill with key splits and their merge in F16 and F32, the prefill kernel
on 8- and 2-token pages read in place, the page repack)
replay from the graph bit for bit like the eager call.  Serving loops capture their decode step this way to cut
launch overhead; the library makes no allocation, memset or synchronisation on these paths, so capture records
kernels only.

Each graph is replayed several times with the program's own eager work between the replays (the output is
poisoned with NaN and the stream synchronised), and every replay is compared with the eager result.
"""
import ctypes
import math

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


def _ragged(name, dtype, hq, hkv, d, ctx, qlens, page_size=16, seed=11):
    rng = np.random.default_rng(seed)
    seq_lens = (np.array(ctx) + np.array(qlens)).astype(np.int32)
    need = [math.ceil(int(L) / page_size) for L in seq_lens]
    num_pages = sum(need) + 3
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(need), max(need)), np.int32)
    used = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[used:used + n]
        used += n
    return W.Workload(name, dtype, hq, hkv, d, page_size, num_pages, 0.3, seq_lens, np.array(qlens, np.int32), bt,
                      seed)


CASES = {
    "split-and-merge": W.qwen2_05b_batched_decode_f16,
    "f32-split-and-merge": W.qwen2_05b_decode_f32,
    "block-merge": lambda: W.llama3_8b_decode_b64_8k_f16(8),
    "verify-32-row-tiles": W.llama3_8b_spec_verify_f16,
    "prefill-key-splits-f16": lambda: _ragged("prefill f16", "f16", 32, 8, 128, [4000], [130]),
    "prefill-key-splits-f32": lambda: _ragged("prefill f32", "f32", 32, 8, 128, [4000], [130]),
    "prefill-d64-f16": lambda: _ragged("prefill d64", "f16", 14, 2, 64, [2048, 2048], [256, 200]),
    "page-size-5-in-place": lambda: _ragged("page size 5", "f16", 32, 8, 128, [700, 97, 1500], [1, 5, 1],
                                            page_size=5),
    "repacked-page-size-5": lambda: _ragged("page size 5 prefill", "f16", 32, 8, 128, [700, 300], [1, 100],
                                            page_size=5),
    "prefill-token-pages-8": lambda: _ragged("page size 8 prefill", "f16", 32, 8, 128, [700, 300], [1, 100],
                                             page_size=8),
    "prefill-token-pages-2-key-splits-f32": lambda: _ragged("page size 2 prefill f32", "f32", 32, 8, 128, [4000],
                                                            [130], page_size=2),
    "head-dim-96-f32": lambda: _ragged("head_dim 96", "f32", 32, 8, 96, [700, 97, 1500], [1, 5, 40]),
}


@pytest.mark.parametrize("noalloc", [False, True], ids=["workspace", "noalloc"])
@pytest.mark.parametrize("case", list(CASES))
def test_captured_call_replays_bit_for_bit(case, noalloc):
    w = CASES[case]()
    t = W.device_tensors(w, None, seed=13)
    lib = M.load_library()
    out = torch.full_like(t["q"], float("nan"))
    a = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out,
                    max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    need = M.workspace_size(a)
    ws = None
    if not noalloc and need:
        ws = M.new_workspace(need, "cuda")
        a.workspace, a.workspace_bytes = ws.data_ptr(), need
    call = lib.mvr_paged_attention_noalloc if noalloc else lib.mvr_paged_attention
    if noalloc and need > M.NOALLOC_SCRATCH_BYTES:
        pytest.skip("larger than the static scratch")

    def launch():
        rc = call(ctypes.byref(a))
        assert rc == 0, lib.mvr_last_error().decode()

    launch()  # eager reference (also settles any per-device set-up before capture)
    torch.cuda.synchronize()
    ref = out.clone()
    assert not torch.isnan(ref).any()

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()  # default priority
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        a.stream = s.cuda_stream
        with torch.cuda.graph(g, stream=s):
            launch()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    print(f"{case} ({'noalloc' if noalloc else 'workspace'}): workspace {need} bytes", flush=True)
    for rep in range(3):
        out.fill_(float("nan"))  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager call"
    del g
    torch.cuda.synchronize()
