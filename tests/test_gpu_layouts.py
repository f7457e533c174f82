"""GPU parity for the layouts and dtypes the other parity tests leave out, through the C ABI against the oracle.

* token-major Q/O (q_stride_head = D, q_stride_token = Hq * D: the packed [1, packed_q_len, Hq * D] layout that
  forward_attention transposes the output into, common.rs:326-332) on every kernel path: split context with the
  partition merge, the block-merge launch, 32-row verify tiles and the chunked-prefill kernel;
* the request-level entry mvr_forward_paged_attention (common.rs:426-464 + :739-817) against the oracle's
  request-level restatement, not against the batched call;
* F32, the activation dtype the reference's GPU backends force (server/mod.rs:505-530), at prefill size (q_len 256,
  D 128) and at decode batch 16 x 8K (D 128);
* the batch one scheduler step emits (scheduler.rs:258-271): 63 decodes at 8K and one 256-token prefill chunk.

Bar: max-abs 1e-5 (F32) and 2e-3 (F16) against the oracle's reference dataflow.
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


def oracle_out(w, vals):
    q, k, v = vals
    return O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                             w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)


def ragged(name, seed, dtype, hq, hkv, d, seq_lens, q_lens, page_size=16):
    rng = np.random.default_rng(seed)
    seq_lens = np.asarray(seq_lens, np.int32)
    n = [math.ceil(int(L) / page_size) for L in seq_lens]
    num_pages = sum(n) + 3
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(seq_lens), max(n)), np.int32)
    used = 0
    for s in range(len(seq_lens)):
        bt[s, :n[s]] = perm[used:used + n[s]]
        used += n[s]
    return W.Workload(name, dtype, hq, hkv, d, page_size, num_pages, 0.3, seq_lens, np.asarray(q_lens, np.int32), bt,
                      seed)


def token_major_cases():
    return {
        # 8 ragged Qwen2-0.5B sequences: context partitions merged by merge_partitions_kernel
        "split+merge": W.qwen2_05b_batched_decode_f16,
        # 64 uniform 1K-token Llama-3-8B sequences: 4 partitions per tile, merged in LDS (block-merge launch)
        "block-merge": lambda: ragged("uniform 64 x 1024", 71, "f16", 32, 8, 128, [1024] * 64, [1] * 64),
        # ragged 5-token verify rows (32-row tiles), F32
        "verify f32": lambda: ragged("verify f32", 72, "f32", 32, 8, 128, [1500, 777, 3000, 64], [5, 5, 5, 5]),
        # the Qwen2-7B chunked-prefill shape: the prefill kernel
        "prefill": W.qwen2_7b_chunked_prefill_f16,
    }


@pytest.mark.parametrize("case", list(token_major_cases()))
def test_token_major_q_and_out_match_oracle(case):
    w = token_major_cases()[case]()
    say(f"[token-major] {case}: {w.name}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    # [total_q, Hq, D] in memory, seen as [Hq, total_q, D]: stride_head = D, stride_token = Hq * D.
    q_tm = t["q"].permute(1, 0, 2).contiguous().permute(1, 0, 2)
    assert q_tm.stride() == (w.head_dim, w.num_q_heads * w.head_dim, 1)
    out_tm = torch.full((w.total_q, w.num_q_heads, w.head_dim), float("nan"), dtype=q_tm.dtype,
                        device="cuda").permute(1, 0, 2)
    args = M.make_args(q_tm, t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out_tm,
                       max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    if case == "block-merge":
        assert M.workspace_size(args) == 0  # planned as the block-merge launch: no partials
    M.paged_attention(q_tm, t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out_tm,
                      max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    head_major = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                                   t["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len,
                                   sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    got = out_tm.float().cpu().numpy()
    ref = oracle_out(w, vals)
    err = float(np.abs(got - ref).max())
    say(f"[token-major] {case}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[w.dtype], err
    # Same plan, same arithmetic: only the addresses differ, so the bits match the head-major call.
    assert torch.equal(out_tm, head_major)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("page_size,cached,q_len", [(16, 4095, 1), (16, 1000, 5), (16, 1800, 200), (3, 40, 7),
                                                    (32, 0, 96)])
def test_request_level_entry_matches_oracle(dtype, page_size, cached, q_len):
    """mvr_forward_paged_attention with the reference's PagedCacheLayout (page ids in logical order, a partial last
    page) against oracle_forward_paged_attention, the oracle's restatement of forward_cpu_paged_attention +
    forward_paged_attention, not against another HIP call."""
    hq, hkv, d = 28, 4, 128
    L = cached + q_len
    n = math.ceil(L / page_size)
    rng = np.random.default_rng(1000 + page_size + cached + q_len + (dtype == "f32"))
    npd = np.float16 if dtype == "f16" else np.float32
    num_pages = n + 5
    kp = (rng.standard_normal((num_pages, 1, hkv, page_size, d)) * 0.3).astype(npd)
    vp = (rng.standard_normal((num_pages, 1, hkv, page_size, d)) * 0.3).astype(npd)
    ids = rng.permutation(num_pages)[:n].astype(np.int32)
    q = (rng.standard_normal((1, hq, q_len, d)) * 0.3).astype(npd)
    lay = M.PagedCacheLayout(torch.from_numpy(kp).cuda(), torch.from_numpy(vp).cuda(), torch.from_numpy(ids).cuda(),
                             page_size, L)
    y = M.forward_paged_attention(torch.from_numpy(q).cuda(), lay, hq, hkv, d, cached, q_len)
    torch.cuda.synchronize()
    ref = O.forward_paged_attention(q, kp, vp, ids.astype(np.int64), page_size, L, hq, hkv, d, cached, q_len,
                                    dtype=O.F16 if dtype == "f16" else O.F32)
    got = y[0].float().cpu().numpy()
    err = float(np.abs(got - ref).max())
    say(f"[request-level] {dtype} P={page_size} c={cached} q={q_len}: max-abs vs oracle {err:.3e}")
    assert y.shape == (1, hq, q_len, d) and y.dtype == lay.key_pool.dtype
    assert err <= TOL[dtype], err


@pytest.mark.parametrize("make", [
    lambda: W.qwen2_7b_chunked_prefill_f16("f32"),        # q_len 256, D 128: the prefill kernel's F32 tile
    lambda: W.llama3_8b_decode_b64_8k_f16(16, "f32"),     # decode, batch 16 x 8K, D 128
], ids=["prefill-256-d128", "decode-b16-8k-d128"])
def test_f32_at_serving_scale_matches_oracle(make):
    w = make()
    say(f"[f32] {w.name}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    out = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                            max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    ref = oracle_out(w, vals)
    err = float(np.abs(got - ref).max())
    say(f"[f32] {w.name}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= 1e-5, err


def test_mixed_decode_and_prefill_batch_matches_oracle():
    """63 decodes over 8K tokens and one 256-token chunk on a 2K prefix in one call, the order a scheduler step
    packs them (decodes first, scheduler.rs:258-271): with and without the host copies of the lengths that let the
    planner route each sequence to its kernel."""
    w = W.llama3_8b_mixed_decode_prefill_f16()
    say(f"[mixed] {w.name}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    ref = oracle_out(w, vals)
    outs = []
    for hints in (False, True):
        kw = dict(cu_q_lens_host=w.cu_q_lens, seq_lens_host=w.seq_lens) if hints else {}
        out = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                                t["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len,
                                sum_seq_lens=int(w.seq_lens.sum()), **kw)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        err = float(np.abs(got - ref).max())
        say(f"[mixed] host hints {hints}: max-abs vs oracle {err:.3e}")
        assert np.isfinite(got).all() and err <= 2e-3, (hints, err)
        outs.append(out)
