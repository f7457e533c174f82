"""GPU parity for batches that mix decode-sized and prefill-sized requests in any order (scheduler.rs:258-271 packs
the decodes first; other callers need not), through the C ABI against the oracle.

A call whose longest query is prefill-sized runs as two launches: the split-context kernel over the range of
sequences that holds the decode class, computing those of its sequences whose device q_len fits its plan, and the
prefill kernel over every sequence, computing all the others.  The host copies of the length tables only shape the
two plans, so the output must match the oracle with them, without them, and with hints that disagree with the
device tables (stale copies): a wrong hint may cost speed, never rows.  The classes are interleaved here (prefill,
decode, prefill, decode, ...) so that each launch skips sequences inside its own range, on the block-merge, dense
and split-context plans of the decode class and on the prefill kernel with and without key splits.

Bar: max-abs 1e-5 (F32) and 2e-3 (F16) against the oracle's reference dataflow (common.rs:739-817).
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


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()
    O.build()


def interleaved(name, seed, dtype, hq, hkv, d, decode_lens, prefills, page_size=16, decode_q=None):
    """Decode sequences (contexts decode_lens, q_len 1 or decode_q[i]) with prefill chunks (cached, q_len)
    inserted at every other position from the front: prefill, decode, prefill, decode, ..., then the remaining
    decodes."""
    seq_lens, q_lens = [], []
    dec = list(zip(decode_lens, decode_q if decode_q is not None else [1] * len(decode_lens)))
    for cached, q in prefills:
        seq_lens.append(cached + q)
        q_lens.append(q)
        if dec:
            L, qd = dec.pop(0)
            seq_lens.append(int(L))
            q_lens.append(int(qd))
    seq_lens += [int(L) for L, _ in dec]
    q_lens += [int(qd) for _, qd in dec]
    rng = np.random.default_rng(seed)
    n = [math.ceil(int(L) / page_size) for L in seq_lens]
    num_pages = sum(n) + 3
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(seq_lens), max(n)), np.int32)
    used = 0
    for s in range(len(seq_lens)):
        bt[s, :n[s]] = perm[used:used + n[s]]
        used += n[s]
    return W.Workload(name, dtype, hq, hkv, d, page_size, num_pages, 0.3, np.asarray(seq_lens, np.int32),
                      np.asarray(q_lens, np.int32), bt, seed)


def cases():
    rng = np.random.default_rng(77)
    return {
        # decode class: 64 uniform 1K-token Llama-3-8B sequences (with hints: the block-merge launch)
        "f16-block-merge": lambda: interleaved("mixed f16 64 x 1024 + 3 chunks", 81, "f16", 32, 8, 128,
                                               [1024] * 64, [(700, 96), (0, 200), (1500, 33)]),
        # decode class: 40 ragged sequences (with hints: the dense layout)
        "f16-dense": lambda: interleaved("mixed f16 40 ragged + 2 chunks", 82, "f16", 32, 8, 128,
                                         list(rng.integers(128, 4097, 40)), [(2048, 256), (300, 130)]),
        # Qwen2-0.5B shape (G = 7): split-context decode with the partition merge
        "f16-qwen2-split": lambda: interleaved("mixed f16 qwen2 8 ragged + 2 chunks", 83, "f16", 14, 2, 64,
                                               list(rng.integers(128, 4097, 8)), [(512, 64), (0, 100)]),
        # decodes (q_len 1) and speculative verification rows (q_len 5, 20 grouped rows) in the small class
        "f16-verify-decode": lambda: interleaved("mixed f16 verify + decode + 2 chunks", 85, "f16", 32, 8, 128,
                                                 list(rng.integers(1024, 8193, 10)), [(1000, 300), (64, 64)],
                                                 decode_q=[5, 1] * 5),
        # F32 (the reference's GPU backends' activation dtype)
        "f32-split": lambda: interleaved("mixed f32 12 ragged + 2 chunks", 84, "f32", 32, 8, 128,
                                         list(rng.integers(100, 2049, 12)), [(600, 80), (0, 150)]),
    }


def stale(w):
    """Host copies that disagree with the device tables but stay within the call's bounds: every sequence
    claims the previous sequence's (q_len, seq_len), so the classes move to other sequences."""
    q = np.roll(w.q_lens, 1)
    sl = np.maximum(np.roll(w.seq_lens, 1), q).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(q)]).astype(np.int32)
    return dict(seq_lens_host=sl, cu_q_lens_host=cu)


@pytest.mark.parametrize("case", list(cases()))
def test_interleaved_classes_match_oracle(case):
    w = cases()[case]()
    say(f"[mixed] {case}: {w.name}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    ref = O.paged_attention(vals[0], vals[1], vals[2], w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads,
                            w.num_kv_heads, w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32,
                            num_threads=16)
    variants = {
        "no hints": {},
        "hints": dict(seq_lens_host=w.seq_lens, cu_q_lens_host=w.cu_q_lens),
        "cu hint only": dict(cu_q_lens_host=w.cu_q_lens),
        "stale hints": stale(w),
    }
    for label, kw in variants.items():
        out = torch.full((w.num_q_heads, w.total_q, w.head_dim), float("nan"), dtype=t["q"].dtype, device="cuda")
        M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                          out, max_q_len=w.max_q_len, max_seq_len=w.max_seq_len,
                          sum_seq_lens=int(w.seq_lens.sum()), **kw)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        err = float(np.abs(got - ref).max()) if np.isfinite(got).all() else float("inf")
        say(f"[mixed] {case} {label}: max-abs vs oracle {err:.3e}")
        # every row written (the output starts as NaN) and within tolerance
        assert np.isfinite(got).all(), (label, int(np.isnan(got).sum()))
        assert err <= TOL[w.dtype], (label, err)
