"""GPU parity of cascade (prefix-sharing) attention, mvr_paged_attention_cascade.

Groups of consecutive sequences share their first pages; the prefix is attended once per group and merged with
each member's suffix.  The result is the same attention (an exact split of the softmax sum), so the bar is the
plain call's: 2e-3 (F16) / 1e-5 (F32) against the oracle, which knows nothing of the groups.  Covers the
speculative-verification workload's own groups (4 x 4 sequences sharing 1024 tokens), ragged groups with a lone
sequence and a group of one, a prefix pass that takes the chunked-prefill kernel (many rows per group), F32 and
head dimensions 64, 96, 160 and 256 (the last three with both passes on the split-context kernel), a call with no
group at all, and a decode batch of 64 sequences sharing one 8192-token prompt (plain call checked too).  With
the sum_prefix_lens hint, the verification workload (shared reads 9% of the key reads) runs as the plain call,
bit for bit, and the shared prompt (86%) still cascades.
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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_cascade(w, t, groups, prefix_of_seq, hint=False):
    """groups: consecutive (first_seq, n_seqs, prefix_len) from sequence 0 on; prefix 0 = a member shares nothing.
    Without the sum_prefix_lens hint (the default here) the library always takes the cascade path; with it, a call
    whose shared reads are a small part of its key reads runs as the plain call."""
    cu = w.cu_q_lens
    gcu = np.array([cu[g[0]] for g in groups] + ([cu[groups[-1][0] + groups[-1][1]]] if groups else [0]), np.int32)
    gpre = np.array([g[2] for g in groups], np.int32)
    gbt = np.stack([w.block_tables[g[0]] for g in groups]).astype(np.int32) if groups else None
    spre = np.asarray(prefix_of_seq, np.int32)
    max_gq = max((int(cu[g[0] + g[1]] - cu[g[0]]) for g in groups), default=1)
    max_pre = max((g[2] for g in groups), default=1)
    G = M.make_cascade_groups(dev(gcu) if groups else None, dev(gpre) if groups else None,
                              dev(gbt) if groups else None, dev(spre), max_group_q_len=max_gq,
                              max_prefix_len=max_pre, sum_prefix_lens=int(spre.sum()) if hint else 0)
    args = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                       t["q"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len)
    M.validate_cascade(args, G, w.block_tables, w.seq_lens, cu, gcu if groups else None, gpre if groups else None,
                       gbt, spre)
    keep = (gcu, gpre, gbt, spre)  # noqa: F841 (device copies were made from these)
    out = M.paged_attention_cascade(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                                    t["cu_q_lens"], G, max_q_len=w.max_q_len, max_seq_len=w.max_seq_len,
                                    sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def check(w, vals, got, tag):
    q, k, v = vals
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got - ref).max())
    say(f"[cascade] {tag}: max-abs vs oracle {err:.3e}")
    assert err <= TOL[w.dtype], err


def test_spec_verify_groups_match_oracle():
    w = W.llama3_8b_spec_verify_f16()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    groups = [(4 * g, 4, 1024) for g in range(4)]
    got = run_cascade(w, t, groups, [1024] * 16)
    check(w, vals, got, "spec-verify, 4 groups x 4 sequences, 1024-token prefixes")


def test_shared_prompt_decode_matches_oracle():
    # 64 decode sequences share one 8192-token prompt (a single group of 64: 256 grouped rows, so the prefix
    # pass takes the chunked-prefill kernel), then private contexts of 256..2048 tokens; the plain call on
    # the same tensors is checked too.
    w = W.llama3_8b_shared_prompt_decode_f16()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    got = run_cascade(w, t, [(0, w.num_seqs, 8192)], [8192] * w.num_seqs)
    check(w, vals, got, "shared prompt, 64 sequences x 8192-token prefix")
    plain = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                              t["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len,
                              sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    check(w, vals, plain.float().cpu().numpy(), "shared prompt, plain call")


def shared_prefix_workload(dtype, d, page_size, q_lens, cached, groups, hq=8, hkv=2, seed=3):
    """Sequences with the given q_lens / cached lengths; members of each (first, n, prefix) group share their first
    prefix // page_size pages."""
    rng = np.random.default_rng(seed)
    q_lens = np.asarray(q_lens, np.int32)
    seq_lens = (np.asarray(cached, np.int32) + q_lens).astype(np.int32)
    need = [math.ceil(int(L) / page_size) for L in seq_lens]
    num_pages = sum(need) + 8
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(need), max(need)), np.int32)
    used = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[used:used + n]
        used += n
    shared = 0
    for first, n, pre in groups:
        for s in range(first + 1, first + n):  # members after the first adopt its prefix pages
            bt[s, :pre // page_size] = bt[first, :pre // page_size]
            shared += pre // page_size
    wk = W.Workload("shared-prefix test", dtype, hq, hkv, d, page_size, num_pages, 0.5, seq_lens, q_lens, bt, seed,
                    shared_pages=shared)
    return wk


@pytest.mark.parametrize("dtype,d", [("f16", 128), ("f16", 64), ("f32", 64), ("f32", 128), ("f16", 96), ("f32", 160),
                                     ("f16", 256)])
def test_ragged_groups_match_oracle(dtype, d):
    # groups: seqs 0-2 share 48 tokens, seq 3 shares nothing (prefix-0 group), seqs 4-5 share 32, seq 6 is a group
    # of one (prefix 64), seq 7 follows the last group
    q_lens = [1, 5, 3, 1, 17, 2, 4, 6]
    cached = [300, 48, 100, 77, 40, 200, 64, 90]
    groups = [(0, 3, 48), (3, 1, 0), (4, 2, 32), (6, 1, 64)]
    prefix = [48, 48, 48, 0, 32, 32, 64, 0]
    w = shared_prefix_workload(dtype, d, 16, q_lens, cached, groups)
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    got = run_cascade(w, t, groups, prefix)
    check(w, vals, got, f"ragged groups {dtype} D={d}")


@pytest.mark.parametrize("d", [128, 96])
def test_prefix_pass_on_the_prefill_kernel(d):
    # 2 x 40 query tokens x 4 heads per KV head = 320 rows share a 512-token prefix: the prefix pass is a dense
    # contraction and takes the chunked-prefill kernel; the suffix pass stays on the split-context kernel.
    q_lens = [40, 40, 3]
    cached = [600, 512, 900]
    groups = [(0, 2, 512)]
    w = shared_prefix_workload("f16", d, 16, q_lens, cached, groups, hq=16, hkv=4, seed=9)
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    got = run_cascade(w, t, groups, [512, 512, 0])
    check(w, vals, got, f"prefill-kernel prefix pass D={d}")


def test_no_groups_equals_plain_call():
    w = W.qwen2_05b_batched_decode_f16()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    got = run_cascade(w, t, [], [0] * w.num_seqs)
    check(w, vals, got, "no groups")


def test_small_sharing_runs_as_the_plain_call():
    # The verification workload's 4 groups share 1024 tokens each: 12288 of ~139K key reads saved, below the 25%
    # that the cascade needs to pay, so with the hint the call is the plain call (the same launches, same bits).
    w = W.llama3_8b_spec_verify_f16()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    got = run_cascade(w, t, [(4 * g, 4, 1024) for g in range(4)], [1024] * 16, hint=True)
    plain = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                              t["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len,
                              sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    assert np.array_equal(got, plain.float().cpu().numpy())
    check(w, vals, got, "spec-verify with the sharing hint (plain path)")


def test_large_sharing_still_cascades():
    w = W.llama3_8b_shared_prompt_decode_f16()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    got = run_cascade(w, t, [(0, w.num_seqs, 8192)], [8192] * w.num_seqs, hint=True)
    check(w, vals, got, "shared prompt with the sharing hint (cascade path)")
