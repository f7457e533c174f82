"""GPU parity on seeded random batches: the planner's choices (split-context plans, block merge, dense layout,
deep pipeline, token pages, the prefill kernel with key splits, the two launches of a mixed batch, the repack)
follow from the batch's shape, so a sweep over shapes reaches combinations that the hand-written cases do not.

Each case draws: F16 or F32; (Hq, Hkv, D) from the shapes of the reference's target and draft models
(Qwen2.5-0.5B 14/2/64, Qwen2.5-1.5B 12/2/128, Qwen2.5-7B 28/4/128, Llama-3.2-1B 32/8/64, Llama-3.2-3B
24/8/128, Llama-3.1-8B 32/8/128) and five others (8/8/64, 16/2/128, and the head dimensions 96, 32 and 256 as
16/2/96, 12/4/32 and 8/4/256); 1-80 sequences; per sequence a cached length and a query length (decodes,
verification rows, prefill chunks, in any order); a page size from 1 to 48; and how the host hints are passed
(none, both tables, only cu_q_lens, stale copies).  The output starts as NaN and must be finite everywhere and
within 2e-3 (F16) / 1e-5 (F32) of the oracle.  Sizes stay small enough for the oracle to run in well under a
second per case.
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
SHAPES = [(14, 2, 64), (12, 2, 128), (28, 4, 128), (32, 8, 64), (24, 8, 128), (32, 8, 128), (8, 8, 64), (16, 2, 128),
          (16, 2, 96), (12, 4, 32), (8, 4, 256)]
PAGES = [1, 2, 3, 5, 8, 16, 16, 16, 24, 32, 48]
HINTS = ["none", "both", "cu", "stale"]
N_CASES = 200


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()
    O.build()


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    dtype = "f16" if rng.random() < 0.7 else "f32"
    hq, hkv, d = SHAPES[rng.integers(len(SHAPES))]
    kind = rng.choice(["decode", "verify", "prefill", "mixed"])
    n = int(rng.choice([1, 2, 3, 5, 8] if kind == "prefill" else [1, 2, 3, 5, 8, 16, 33, 64, 80]))
    q_lens, cached = [], []
    n_prefill = 0
    for _ in range(n):
        k = kind if kind != "mixed" else rng.choice(["decode", "decode", "verify", "prefill"])
        if k == "prefill":
            n_prefill += 1
            k = k if n_prefill <= 3 or kind == "prefill" else "decode"
        q = 1 if k == "decode" else int(rng.integers(2, 7)) if k == "verify" else int(rng.integers(17, 300))
        c = int(rng.integers(0, 3000 if k == "prefill" else 9000))
        q_lens.append(q)
        cached.append(c)
    # shrink the contexts until the oracle's work (query-key pairs x heads x head_dim) is at most ~4e8
    budget = 4e8 / (hq * d)
    scale = 1.0
    while sum(q * (c * scale + q) for q, c in zip(q_lens, cached)) > budget and scale > 0.01:
        scale *= 0.7
    cached = [int(c * scale) for c in cached]
    seq_lens = np.array([c + q for c, q in zip(cached, q_lens)], np.int32)
    page = int(rng.choice(PAGES))
    need = [math.ceil(int(L) / page) for L in seq_lens]
    num_pages = sum(need) + 5
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((n, max(need) + int(rng.integers(0, 3))), np.int32)
    used = 0
    for s in range(n):
        bt[s, :need[s]] = perm[used:used + need[s]]
        used += need[s]
    hints = HINTS[int(rng.integers(len(HINTS)))]
    w = W.Workload(f"random {seed}", dtype, hq, hkv, d, page, num_pages, 0.3, seq_lens, np.array(q_lens, np.int32),
                   bt, 2000 + seed)
    return w, hints


@pytest.mark.parametrize("seed", range(N_CASES))
def test_random_batch_matches_oracle(seed):
    w, hints = draw(seed)
    say(f"[random {seed}] {w.dtype} Hq {w.num_q_heads} Hkv {w.num_kv_heads} D {w.head_dim} page {w.page_size} "
        f"seqs {w.num_seqs} q {w.q_lens.tolist()[:12]} seq {w.seq_lens.tolist()[:12]} hints {hints}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    kw = {}
    if hints == "both":
        kw = dict(seq_lens_host=w.seq_lens, cu_q_lens_host=w.cu_q_lens)
    elif hints == "cu":
        kw = dict(cu_q_lens_host=w.cu_q_lens)
    elif hints == "stale":
        q = np.roll(w.q_lens, 1)
        kw = dict(seq_lens_host=np.maximum(np.roll(w.seq_lens, 1), q).astype(np.int32),
                  cu_q_lens_host=np.concatenate([[0], np.cumsum(q)]).astype(np.int32))
    out = torch.full((w.num_q_heads, w.total_q, w.head_dim), float("nan"), dtype=t["q"].dtype, device="cuda")
    M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out,
                      max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()), **kw)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = O.paged_attention(vals[0], vals[1], vals[2], w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads,
                            w.num_kv_heads, w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32,
                            num_threads=16)
    finite = bool(np.isfinite(got).all())
    err = float(np.abs(got - ref).max()) if finite else float("inf")
    say(f"[random {seed}] max-abs vs oracle {err:.3e}")
    assert finite and err <= TOL[w.dtype], err
