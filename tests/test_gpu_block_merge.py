"""GPU parity of the block-merge launch of the split-context kernel.

When a uniform batch splits every context into exactly one block's worth of
partitions (4), the planner puts the partitions of one (sequence, KV head)
in one block and merges them through LDS instead of writing fp32 partials
and launching the merge kernel.  The plan is visible from the host: such a
call needs no workspace.  Same bar as every call: 2e-3 (F16) / 1e-5 (F32)
against the oracle.  Covers F16 at head_dim 128 (the batch-64 decode shape at
1K tokens), ragged lengths planned as uniform (no length hint), so that short
sequences leave partitions without keys that still join the block's merge,
and F32 at head_dim 64.
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


def decode_workload(name, dtype, hq, hkv, d, lens, seed, page_size=16):
    rng = np.random.default_rng(seed)
    seq_lens = np.asarray(lens, np.int32)
    need = [math.ceil(int(L) / page_size) for L in seq_lens]
    num_pages = sum(need) + 4
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(need), max(need)), np.int32)
    used = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[used:used + n]
        used += n
    return W.Workload(name, dtype, hq, hkv, d, page_size, num_pages, 0.3, seq_lens, np.ones(len(need), np.int32), bt,
                      seed)


def run_and_check(w, hint):
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    sum_hint = int(w.seq_lens.sum()) if hint else 0
    args = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                       t["q"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=sum_hint)
    assert M.workspace_size(args) == 0, "expected the block-merge plan (no workspace)"
    out = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                            max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=sum_hint)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    q, k, v = vals
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got - ref).max())
    say(f"[block-merge] {w.name}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[w.dtype], err


def test_uniform_f16_d128():
    run_and_check(decode_workload("f16 D128 64 x 1024", "f16", 32, 8, 128, [1024] * 64, 61), hint=True)


def test_ragged_lengths_planned_uniform():
    rng = np.random.default_rng(62)
    lens = rng.integers(16, 1024, size=64, endpoint=True)
    lens[0] = 1024  # max_seq_len 1024: 4 partitions of 256 tokens, most sequences leave some without keys
    run_and_check(decode_workload("f16 D128 64 x U[16,1024] without hint", "f16", 32, 8, 128, lens, 62), hint=False)


def test_uniform_f32_d64():
    run_and_check(decode_workload("f32 D64 256 x 512", "f32", 14, 2, 64, [512] * 256, 63), hint=True)
