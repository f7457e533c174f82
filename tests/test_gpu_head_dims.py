"""GPU parity at the head dimensions besides 64 and 128: every multiple of 32 up to 256, F16 and F32.

The reference's attention takes any head dimension (AttentionDimensions, common.rs:189-206); its own Qwen2 and
Llama shapes use 64 and 128, which keep every plan.  The others run the split-context kernel with 16-row tiles in
1-wavefront blocks and the merge pass, and prefill-sized calls the prefill kernel (rows of more than 128 elements
in blocks of one wavefront group), so each is checked on the call shapes that reach different parts of them: a
ragged decode batch (partials merged across partitions), verification rows (two row tiles per KV head), a
prefill-sized call (causal limits inside the query), a mixed batch in 5-token pages (the repack into 16-token
pages, with host hints), one long context (more than 64 partitions: the merge's wide rounds) and a chunk on a
long context (the prefill kernel's key splits and their merge).  Output starts as NaN and must be finite
everywhere and within 2e-3 (F16) / 1e-5 (F32) of the oracle.
"""
import math
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mvr_attn as M  # noqa: E402
import oracle as O  # noqa: E402
import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-5, "f16": 2e-3}
HEAD_DIMS = [32, 96, 160, 192, 224, 256]
# name: (q_lens, cached lengths, page size, host hints)
CASES = {
    "decode-ragged": ([1, 1, 1, 1, 1], [0, 16, 299, 999, 2048], 16, "both"),
    "verify": ([5, 5, 5], [35, 695, 1495], 32, "none"),
    "prefill": ([40, 70], [100, 300], 16, "cu"),
    "mixed-repacked": ([1, 1, 37, 1], [500, 20, 100, 900], 5, "both"),
    "long-context": ([1], [19999], 16, "none"),
    "prefill-key-splits": ([64], [8000], 32, "none"),
}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()
    O.build()


def workload(dtype, d, q_lens, cached, page, seed):
    rng = np.random.default_rng(seed)
    q_lens = np.asarray(q_lens, np.int32)
    seq_lens = (np.asarray(cached, np.int32) + q_lens).astype(np.int32)
    need = [math.ceil(int(L) / page) for L in seq_lens]
    num_pages = sum(need) + 3
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(need), max(need) + 1), np.int32)
    used = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[used:used + n]
        used += n
    return W.Workload(f"head_dim {d}", dtype, 8, 2, d, page, num_pages, 0.5, seq_lens, q_lens, bt, seed)


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_other_head_dims_match_oracle(dtype, d, case):
    q_lens, cached, page, hints = CASES[case]
    w = workload(dtype, d, q_lens, cached, page, seed=d + len(case))
    say(f"[head_dim {d}] {dtype} {case}: page {page} q {w.q_lens.tolist()} seq {w.seq_lens.tolist()} hints {hints}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    kw = {}
    if hints == "both":
        kw = dict(seq_lens_host=w.seq_lens, cu_q_lens_host=w.cu_q_lens)
    elif hints == "cu":
        kw = dict(cu_q_lens_host=w.cu_q_lens)
    out = torch.full((w.num_q_heads, w.total_q, d), float("nan"), dtype=t["q"].dtype, device="cuda")
    M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out,
                      max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()), **kw)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = O.paged_attention(vals[0], vals[1], vals[2], w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads,
                            w.num_kv_heads, d, page, dtype=O.F16 if dtype == "f16" else O.F32, num_threads=16)
    finite = bool(np.isfinite(got).all())
    err = float(np.abs(got - ref).max()) if finite else float("inf")
    say(f"[head_dim {d}] {dtype} {case}: max-abs vs oracle {err:.3e}")
    assert finite and err <= TOL[dtype], err
