"""GPU parity: the HIP path (through the C ABI) against the oracle.

Bar: max-abs 1e-5 for F32 and 2e-3 for F16 against the oracle's reference
dataflow (common.rs:739-817, per-op dtype rounding); page-table indexing
bit-exact.  Full-size workloads are also checked through size-independent
properties (block-table relocation, poisoned unused slots, determinism).
"""
import ctypes
import json
import math
import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mvr_attn as M  # noqa: E402
import oracle as O  # noqa: E402
import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-5, "f16": 2e-3}
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()
    O.build()


def run_hip(w, t, scale=0.0, hint=True):
    out = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                            max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, scale=scale,
                            sum_seq_lens=int(w.seq_lens.sum()) if hint else 0)
    torch.cuda.synchronize()
    return out


def run_oracle(w, vals, mode=O.REF_CONCAT_V):
    q, k, v = vals
    return O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                             w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, mode=mode,
                             num_threads=16)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_workload_parity_with_oracle(cfg):
    w = W.CONFIGS[cfg]()
    say(f"[parity] config {cfg}: {w.name}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    out = run_hip(w, t).float().cpu().numpy().astype(np.float64)
    ref = run_oracle(w, vals)
    err = np.abs(out - ref).max()
    exact = run_oracle(w, vals, O.EXACT_F64)
    err_exact = np.abs(out - exact).max()
    say(f"[parity] config {cfg}: max-abs vs oracle {err:.3e}, vs f64 {err_exact:.3e}")
    assert np.isfinite(out).all()
    assert err <= TOL[w.dtype], err
    # Without the sum_seq_lens hint the planner may split contexts differently; the result stays in tolerance.
    out2 = run_hip(w, t, hint=False).float().cpu().numpy().astype(np.float64)
    assert np.abs(out2 - ref).max() <= TOL[w.dtype]


def test_reference_unit_tests_on_gpu():
    """common.rs:1031-1141 closed forms, head_dim zero-padded to 64 (zeros add nothing to q.k and give zero output
    columns), keys in 16-token pages with a reversed block table."""
    cases = json.load(open(GOLDEN))["cases"]
    for case in cases:
        if "paged" in case:
            continue
        hq, hkv, d = case["num_q_heads"], case["num_kv_heads"], case["head_dim"]
        c, ql = case["cached_kv_len"], case["q_len"]
        L = c + ql
        dt = torch.float16 if case["dtype"] == "f16" else torch.float32
        D = 64
        q = torch.zeros(hq, ql, D, dtype=dt)
        q[:, :, :d] = torch.tensor(case["q"], dtype=torch.float32).reshape(hq, ql, d).to(dt)
        npages = 3
        kp = torch.zeros(npages, 1, hkv, 16, D, dtype=dt)
        vp = torch.zeros(npages, 1, hkv, 16, D, dtype=dt)
        kk = torch.tensor(case["k"], dtype=torch.float32).reshape(hkv, L, d)
        vv = torch.tensor(case["v"], dtype=torch.float32).reshape(hkv, L, d)
        kp[2, 0, :, :L, :d] = kk.to(dt)
        vp[2, 0, :, :L, :d] = vv.to(dt)
        bt = torch.tensor([[2, 0]], dtype=torch.int32)
        out = M.paged_attention(q.cuda(), kp.cuda(), vp.cuda(), bt.cuda(), torch.tensor([L], dtype=torch.int32).cuda(),
                                torch.tensor([0, ql], dtype=torch.int32).cuda(), max_q_len=ql, max_seq_len=L)
        torch.cuda.synchronize()
        got = out.float().cpu()
        np.testing.assert_allclose(got[:, :, :d].reshape(-1).numpy(), case["expected"], atol=1e-5, rtol=0,
                                   err_msg=case["name"])
        assert (got[:, :, d:] == 0).all()
        assert out.dtype == dt  # common.rs:1095-1123: dtype preserved


@pytest.mark.parametrize("page_size", [3, 16])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_reference_paged_fixture_semantics_on_gpu(dtype, page_size):
    """common.rs:1143-1203: block table [2, 0], GQA 2:1, cached_kv_len 3, q_len 2.  At the fixture's own page
    size 3 (common.rs:1176), tokens 0-2 fill physical page 2 and tokens 3-4 the first slots of page 0, whose last
    slot holds poison 99; at page size 16 all five sit in page 2 with 99 past them.  Pages off the table hold 88.
    F32 must reproduce the fixture's expected output; F16 (inputs rounded to f16) the oracle's."""
    case = [c for c in json.load(open(GOLDEN))["cases"] if "paged" in c][0]
    dt = torch.float16 if dtype == "f16" else torch.float32
    D, P = 64, page_size
    kp = np.full((3, 1, 1, P, D), 88.0, np.float32)
    vp = np.full((3, 1, 1, P, D), 88.0, np.float32)
    k5 = np.array(case["k"], np.float32).reshape(5, 2)
    v5 = np.array(case["v"], np.float32).reshape(5, 2)
    for pool, vals in ((kp, k5), (vp, v5)):
        for page in (2, 0):
            pool[page] = 0.0
        for t in range(5):
            page, slot = (2, 0)[t // P], t % P
            pool[page, 0, 0, slot, :2] = vals[t]
        for t in range(5, 2 * P):
            pool[(2, 0)[t // P], 0, 0, t % P] = 99.0  # unused slots of the table's pages
    q = np.zeros((2, 2, D), np.float32)
    q[:, :, :2] = np.array(case["q"], np.float32).reshape(2, 2, 2)
    bt = np.array([[2, 0]], np.int32)
    out = M.paged_attention(torch.from_numpy(q).to(dt).cuda(), torch.from_numpy(kp).to(dt).cuda(),
                            torch.from_numpy(vp).to(dt).cuda(), torch.from_numpy(bt).cuda(),
                            torch.tensor([5], dtype=torch.int32).cuda(), torch.tensor([0, 2], dtype=torch.int32).cuda(),
                            max_q_len=2, max_seq_len=5, scale=1.0 / math.sqrt(2.0))  # the fixture's head_dim is 2
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert (got[:, :, 2:] == 0).all()
    if dtype == "f32":
        np.testing.assert_allclose(got[:, :, :2].reshape(-1), case["expected"], atol=1e-5, rtol=0)
    else:
        args = (q[None, :, :, :2].astype(np.float16), kp[..., :2].astype(np.float16), vp[..., :2].astype(np.float16),
                [2, 0][:math.ceil(5 / P)], P, 5, 2, 1, 2, 3, 2)
        ref = O.forward_paged_attention(*args, dtype=O.F16)
        exact = O.forward_paged_attention(*args, dtype=O.F16, mode=O.EXACT_F64)
        # Outputs here are 4..6, where one f16 ulp is 3.9e-3: the 2e-3 bar scales with |output| above 1.
        np.testing.assert_allclose(got[:, :, :2], ref, atol=2e-3, rtol=2e-3)
        # fp32 accumulation then one rounding: within half an f16 ulp of the exact answer (plus fp32 noise).
        half_ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64) / 2
        assert (np.abs(got[:, :, :2] - exact) <= half_ulp + 1e-5).all()


def test_request_level_entry_matches_batched():
    w = W.qwen2_05b_batched_decode_f16()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    batched = run_hip(w, t)
    for s in range(w.num_seqs):
        L = int(w.seq_lens[s])
        n = math.ceil(L / w.page_size)
        lay = M.PagedCacheLayout(t["key_pool"], t["value_pool"], t["block_tables"][s, :n].contiguous(), w.page_size, L)
        rq = t["q"][:, s:s + 1].unsqueeze(0)
        y = M.forward_paged_attention(rq, lay, w.num_q_heads, w.num_kv_heads, w.head_dim, L - 1, 1)
        torch.cuda.synchronize()
        # The context split depends on the whole batch, so the two calls may
        # round their partial sums at different partition boundaries: equal
        # to the F16 bar, not bit for bit.
        diff = (y[0].float() - batched[:, s:s + 1].float()).abs().max().item()
        assert diff <= 2e-3, (s, diff)


def test_one_hot_gather_is_bit_exact():
    """Page-table indexing: each query row's softmax is one-hot on a chosen logical key, so the output must equal
    that key's V row bit for bit (V rows encode page, slot, head and dim as exact integers)."""
    rng = np.random.default_rng(21)
    for dtype in ("f16", "f32"):
        hq, hkv, D, P, N = 8, 2, 64, 16, 40
        seq_lens = np.array([37, 300, 129], np.int32)
        bt = np.zeros((3, 20), np.int32)
        perm = rng.permutation(N)
        used = 0
        for s, L in enumerate(seq_lens):
            n = math.ceil(L / P)
            bt[s, :n] = perm[used:used + n]
            used += n
        kp = np.zeros((N, 1, hkv, P, D), np.float32)
        vp = np.zeros((N, 1, hkv, P, D), np.float32)
        pg, hh, tt, dd = np.meshgrid(np.arange(N), np.arange(hkv), np.arange(P), np.arange(D), indexing="ij")
        vp[:, 0] = (pg * 7 + tt * 3 + hh * 5 + dd) % 1000  # exact in f16
        q = np.zeros((hq, 3, D), np.float32)
        targets = {}
        for s, L in enumerate(seq_lens):
            for h in range(hq):
                j = int(rng.integers(0, L))
                targets[(s, h)] = j
                kvh = h // (hq // hkv)
                e = np.zeros(D, np.float32)
                e[h % (hq // hkv) + 4 * s] = 16.0  # distinct direction per (sequence, query head in group)
                kp[bt[s, j // P], 0, kvh, j % P] += e
                q[h, s] = e
        dt = torch.float16 if dtype == "f16" else torch.float32
        out = M.paged_attention(torch.from_numpy(q).to(dt).cuda(), torch.from_numpy(kp).to(dt).cuda(),
                                torch.from_numpy(vp).to(dt).cuda(), torch.from_numpy(bt).cuda(),
                                torch.from_numpy(seq_lens).cuda(), torch.tensor([0, 1, 2, 3], dtype=torch.int32).cuda(),
                                max_q_len=1, max_seq_len=300, scale=1.0)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        for (s, h), j in targets.items():
            want = vp[bt[s, j // P], 0, h // (hq // hkv), j % P]
            assert np.array_equal(got[h, s], want), (dtype, s, h, j)


def test_workspace_reuse_across_shapes():
    """One uninitialised workspace serves calls of different shapes in any order: outputs repeat bit for bit."""
    cases = [W.qwen2_05b_batched_decode_f16(), W.llama3_8b_spec_verify_f16(), W.qwen2_05b_decode_f32(),
             W.qwen2_7b_chunked_prefill_f16()]
    prepared = []
    need = 0
    for w in cases:
        t = W.device_tensors(w, None, seed=7)
        out = torch.empty_like(t["q"])
        a = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out,
                        max_q_len=w.max_q_len, max_seq_len=w.max_seq_len)
        need = max(need, M.workspace_size(a))
        prepared.append((w, t, out, a))
    ws = M.new_workspace(need, "cuda")
    lib = M.load_library()
    first = {}
    for rnd in range(3):
        for idx in ([0, 1, 2, 3] if rnd != 1 else [3, 1, 0, 2]):
            w, t, out, a = prepared[idx]
            a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
            assert lib.mvr_paged_attention(ctypes.byref(a)) == 0, lib.mvr_last_error()
            torch.cuda.synchronize()
            if idx in first:
                assert torch.equal(first[idx], out), (w.name, rnd)
            else:
                first[idx] = out.clone()
    # fresh per-call workspaces give the same bits (same plan: no sum_seq_lens hint, as above)
    for idx, (w, t, out, a) in enumerate(prepared):
        again = run_hip(w, t, hint=False)
        assert torch.equal(again, first[idx])


@pytest.mark.parametrize("block_merge", ["false", "true"])
def test_many_small_partitions_and_many_tiles(block_merge):
    """16800 (sequence, kv head) tiles, each split into 5-7 partitions of 2 chunks (forced with
    MVR_ATTN_CHUNKS_PER_PARTITION=2, read once per process, hence the child process), planned as uniform: with
    MVR_ATTN_BLOCK_MERGE=false the merge kernel combines many partials per tile, by default each tile is one block of
    8 wavefronts merging in LDS; both match the oracle."""
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    path = os.pathsep.join([os.path.join(root, "mini-vllm-rs_amd"), os.path.join(root, "oracle"),
                            os.environ.get("PYTHONPATH", "")])
    env = dict(os.environ, MVR_ATTN_CHUNKS_PER_PARTITION="2", MVR_ATTN_BLOCK_MERGE=block_merge, PYTHONPATH=path)
    r = subprocess.run([sys.executable, "-u", __file__, "many-partitions-child", block_merge], env=env,
                       capture_output=True, text=True, timeout=300)
    say(r.stdout[-2000:] + r.stderr[-2000:])
    assert r.returncode == 0


def _many_partitions_child(block_merge):
    rng = np.random.default_rng(33)
    B, hq, hkv, D, P = 2100, 8, 8, 64, 16
    seq_lens = rng.integers(130, 200, size=B).astype(np.int32)
    n = [math.ceil(int(L) / P) for L in seq_lens]
    num_pages = sum(n)
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((B, max(n)), np.int32)
    used = 0
    for s in range(B):
        bt[s, :n[s]] = perm[used:used + n[s]]
        used += n[s]
    w = W.Workload("many tiles", "f16", hq, hkv, D, P, num_pages, 0.5, seq_lens, np.ones(B, np.int32), bt, 99)
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    a = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                    torch.empty_like(t["q"]), max_q_len=1, max_seq_len=w.max_seq_len)
    # planned as uniform (no length hint): the two-launch plan keeps fp32 partials in the workspace, the block-merge
    # plan needs none; the two-launch run keeps the length hint (the ragged plan), the block-merge run omits it
    assert (M.workspace_size(a) == 0) == (block_merge == "true")
    out = run_hip(w, t, hint=block_merge == "false").float().cpu().numpy()
    ref = run_oracle(w, vals)
    err = np.abs(out - ref).max()
    print(f"many partitions: {B} sequences x {hkv} kv heads, max-abs vs oracle {err:.3e}", flush=True)
    assert err <= 2e-3


def _ragged_workload(name, seed, hq, hkv, d, ctx, qlens, page_size=16, dtype="f16", scale=0.3):
    rng = np.random.default_rng(seed)
    seq_lens = (np.array(ctx) + np.array(qlens)).astype(np.int32)
    n = [math.ceil(int(L) / page_size) for L in seq_lens]
    num_pages = sum(n) + 5
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(seq_lens), max(n)), np.int32)
    used = 0
    for s in range(len(seq_lens)):
        bt[s, :n[s]] = perm[used:used + n[s]]
        used += n[s]
    return W.Workload(name, dtype, hq, hkv, d, page_size, num_pages, scale, seq_lens,
                      np.array(qlens, np.int32), bt, seed)


@pytest.mark.parametrize("shape", [
    # (hq, hkv, d, cached prefixes, query chunks, page size)
    (28, 4, 128, [2048, 0, 517], [256, 200, 77], 16),   # ragged chunks, one without a prefix
    (8, 2, 64, [300, 1000], [80, 33], 32),              # head_dim 64, page size 32
    (7, 1, 128, [64], [130], 16),                       # a single (sequence, kv head) pair
    (32, 8, 128, [4000, 17, 900], [16, 9, 120], 16),    # decode-sized and prefill-sized requests mixed
    # The kernel's two wavefront groups take alternating 32-token key tiles and merge at the end:
    (28, 4, 128, [0, 31], [16, 33], 16),                # one key tile (the second group sees none), two tiles
    (7, 1, 64, [40], [100], 16),                        # head_dim 64 with an odd number of key tiles
    (32, 8, 128, [0], [1024], 16),                      # a fresh 1,024-token prompt: 8 row tiles of triangular work
    (28, 4, 128, [300, 0, 1000], [256, 128, 384], 16),  # chunks of 1-3 position tiles: tiles ordered by position
    (8, 2, 64, [0, 0], [512, 128], 32),                 # fresh prompts of unequal length, head_dim 64
])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_prefill_shapes_match_oracle(shape, dtype):
    """The chunked-prefill kernel (F16: 32x32x16 products, F32: 32x32x2) on ragged and edge shapes, key splits
    with their merge pass included (the 4000-token case splits its keys in two)."""
    hq, hkv, d, ctx, qlens, P = shape
    w = _ragged_workload("prefill-shape", 41 + sum(qlens), hq, hkv, d, ctx, qlens, page_size=P, dtype=dtype)
    say(f"[prefill] {dtype} {shape}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    out = run_hip(w, t).float().cpu().numpy()
    ref = run_oracle(w, vals)
    err = np.abs(out - ref).max()
    say(f"[prefill] {dtype} {shape}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(out).all() and err <= TOL[dtype], err


@pytest.mark.parametrize("shape", [
    # (hq, hkv, d, cached contexts): few long sequences over few KV heads, whose plans hit the cap of 128
    # partitions per tile and whose merge reads 32 partials per round trip
    (14, 2, 64, [32767]),
    (14, 2, 64, [16383, 9000, 16383, 12000]),
    (32, 8, 128, [32767]),
])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_long_contexts_over_few_heads_match_oracle(shape, dtype):
    hq, hkv, d, ctx = shape
    w = _ragged_workload("long-context", 61 + len(ctx), hq, hkv, d, ctx, [1] * len(ctx), dtype=dtype)
    say(f"[long] {dtype} {shape}")
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    out = run_hip(w, t).float().cpu().numpy()
    ref = run_oracle(w, vals)
    err = np.abs(out - ref).max()
    say(f"[long] {dtype} {shape}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(out).all() and err <= TOL[dtype], err


def test_large_f16_head_dim_64_batch_matches_oracle():
    """64 Qwen2-0.5B-shape sequences of 8,000..10,000 tokens in F16 (about 300 MB of K/V): the planner fills
    three wavefronts per SIMD for such calls, a finer split than smaller ones get."""
    rng = np.random.default_rng(71)
    ctx = [int(x) for x in rng.integers(8000, 10000, size=64)]
    w = _ragged_workload("large-d64", 71, 14, 2, 64, ctx, [1] * 64, dtype="f16")
    assert int(w.seq_lens.sum()) * 2 * 64 * 2 * 2 >= 256 << 20
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    out = run_hip(w, t).float().cpu().numpy()
    ref = run_oracle(w, vals)
    err = np.abs(out - ref).max()
    say(f"[large-d64] max-abs vs oracle {err:.3e}")
    assert np.isfinite(out).all() and err <= TOL["f16"], err


def test_reconstruct_contiguous_matches_reference_gather():
    """paged_cache.rs:363-391 on the device, bit for bit against the oracle's gather: the reference fixture
    (page size 3, table [2, 0], 5 tokens, head_dim 2, F32) and random F16/F32 pools with partial last pages."""
    case = [c for c in json.load(open(GOLDEN))["cases"] if "paged" in c][0]
    pg = case["paged"]
    for name in ("key_pool", "value_pool"):
        pool = np.array(pg[name], np.float32).reshape(pg["page_count"], 1, 1, pg["page_size"], 2)
        got = M.reconstruct_contiguous(torch.from_numpy(pool).cuda(),
                                       torch.tensor(pg["page_ids"], dtype=torch.int32).cuda(), pg["cached_token_count"])
        torch.cuda.synchronize()
        want = O.reconstruct_contiguous(pool, pg["page_ids"], pg["cached_token_count"], dtype=O.F32)
        np.testing.assert_array_equal(got[0].cpu().numpy(), want)
        flat = np.array(case["k" if name == "key_pool" else "v"], np.float32).reshape(1, 5, 2)
        np.testing.assert_array_equal(got[0].cpu().numpy(), flat)  # the fixture's contiguous K/V
    rng = np.random.default_rng(17)
    for dtype, D, P, L in (("f16", 128, 16, 1000), ("f32", 64, 16, 37), ("f16", 64, 32, 65), ("f16", 2, 3, 5)):
        npd = np.float16 if dtype == "f16" else np.float32
        n = math.ceil(L / P) + 3
        pool = rng.standard_normal((n, 1, 4, P, D)).astype(npd)
        ids = rng.permutation(n)[:math.ceil(L / P)].astype(np.int32)
        got = M.reconstruct_contiguous(torch.from_numpy(pool).cuda(), torch.from_numpy(ids).cuda(), L)
        torch.cuda.synchronize()
        want = O.reconstruct_contiguous(pool, ids, L, dtype=O.F16 if dtype == "f16" else O.F32)
        assert np.array_equal(got[0].cpu().numpy().view(np.uint8), want.view(np.uint8)), (dtype, D, P, L)


def test_full_size_properties_decode_b64():
    """Llama-3-8B batch 64 x 8K: relocating every page (and the table with it) and poisoning pages off the table
    leave the output bit-identical; two runs are bit-identical."""
    w = W.llama3_8b_decode_b64_8k_f16()
    say("[props] config 3 full size")
    t = W.device_tensors(w, None)
    a = run_hip(w, t).clone()
    b = run_hip(w, t)
    assert torch.equal(a, b)
    perm = torch.randperm(w.num_pages, generator=torch.Generator().manual_seed(5)).to(torch.int32).cuda()
    k2 = torch.empty_like(t["key_pool"])
    v2 = torch.empty_like(t["value_pool"])
    k2[perm.long()] = t["key_pool"]
    v2[perm.long()] = t["value_pool"]
    del t["key_pool"], t["value_pool"]
    t2 = dict(t, key_pool=k2, value_pool=v2, block_tables=perm[t["block_tables"].long()].contiguous())
    c = run_hip(w, t2)
    assert torch.equal(a, c)


def test_poisoned_tail_slots_and_foreign_pages_are_ignored():
    """Slots past each sequence's length and pages of no table hold NaN/Inf; outputs are unchanged bit for bit."""
    w = W.llama3_8b_spec_verify_f16()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    a = run_hip(w, t).clone()
    k, v = vals[1].copy(), vals[2].copy()
    for s, L in enumerate(w.seq_lens.tolist()):
        last = w.block_tables[s, (L - 1) // w.page_size]
        k[last, 0, :, (L - 1) % w.page_size + 1:] = np.nan
        v[last, 0, :, (L - 1) % w.page_size + 1:] = np.inf
    t2 = W.device_tensors(w, (vals[0], k, v))
    b = run_hip(w, t2)
    assert torch.equal(a, b)


if __name__ == "__main__" and len(sys.argv) > 2 and sys.argv[1] == "many-partitions-child":
    _many_partitions_child(sys.argv[2])


def _same_tokens_two_page_sizes(seed, dtype, hq, hkv, d, seq_lens, q_lens, page_size):
    """The same logical keys and values stored once in page_size-token pages and once in 16-token pages (each with
    its own random page order), with the queries and the two block tables."""
    rng = np.random.default_rng(seed)
    npd = np.float16 if dtype == "f16" else np.float32
    seq_lens = np.asarray(seq_lens, np.int32)
    q = (rng.standard_normal((hq, int(np.sum(q_lens)), d)) * 0.3).astype(npd)
    toks = [(rng.standard_normal((2, int(L), hkv, d)) * 0.3).astype(npd) for L in seq_lens]
    layouts = []
    for P in (page_size, 16):
        need = [math.ceil(int(L) / P) for L in seq_lens]
        n_pages = sum(need) + 3
        perm = rng.permutation(n_pages).astype(np.int32)
        kp = np.full((n_pages, 1, hkv, P, d), 77.0, npd)  # slots past a sequence hold junk
        vp = np.full((n_pages, 1, hkv, P, d), 77.0, npd)
        bt = np.zeros((len(seq_lens), max(need)), np.int32)
        used = 0
        for s, L in enumerate(seq_lens.tolist()):
            bt[s, :need[s]] = perm[used:used + need[s]]
            used += need[s]
            for t in range(L):
                kp[bt[s, t // P], 0, :, t % P] = toks[s][0, t]
                vp[bt[s, t // P], 0, :, t % P] = toks[s][1, t]
        layouts.append((P, kp, vp, bt))
    return q, layouts


@pytest.mark.parametrize("page_size", [1, 2, 3, 5, 8, 24, 40])
@pytest.mark.parametrize("dtype,hq,hkv,d", [("f16", 32, 8, 128), ("f32", 14, 2, 64)])
def test_page_sizes_off_16_match_oracle_and_16_token_pages(page_size, dtype, hq, hkv, d):
    # Decode and verify rows in one ragged batch.  Pages of 2 or more tokens that are not a multiple of 16 are
    # read in place (each token row from its own page), one-token pages repacked into 16-token pages in the
    # workspace; either way the call takes the plan of the 16-token layout, so the result equals the same
    # tokens stored in 16-token pages bit for bit.
    q_lens = [1, 5, 1, 3]
    seq_lens = [37 + page_size, 700, 1 + 2 * page_size, 333]
    q, layouts = _same_tokens_two_page_sizes(900 + page_size, dtype, hq, hkv, d, seq_lens, q_lens, page_size)
    outs = []
    for P, kp, vp, bt in layouts:
        out = M.paged_attention(torch.from_numpy(q).cuda(), torch.from_numpy(kp).cuda(), torch.from_numpy(vp).cuda(),
                                torch.from_numpy(bt).cuda(), torch.tensor(seq_lens, dtype=torch.int32).cuda(),
                                torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32).cuda(),
                                max_q_len=max(q_lens), max_seq_len=max(seq_lens), sum_seq_lens=int(sum(seq_lens)))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    P, kp, vp, bt = layouts[0]
    ref = O.paged_attention(q, kp, vp, bt, np.asarray(seq_lens, np.int32),
                            np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32), hq, hkv, d, P,
                            dtype=O.F16 if dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(outs[0].astype(np.float64) - ref).max())
    view = np.uint16 if dtype == "f16" else np.uint32
    diff = int(np.count_nonzero(outs[0].view(view) != outs[1].view(view)))
    say(f"[page size {page_size}] {dtype} D={d}: max-abs vs oracle {err:.3e}; {diff} outputs differ from 16-token pages")
    assert err <= (2e-3 if dtype == "f16" else 1e-5) and diff == 0


@pytest.mark.parametrize("page_size", [2, 8, 24])
@pytest.mark.parametrize("dtype,hq,hkv,d", [("f16", 32, 8, 128), ("f32", 32, 8, 128), ("f16", 14, 2, 64)])
def test_uniform_batch_in_small_pages_matches_oracle(page_size, dtype, hq, hkv, d):
    # A uniform decode batch, which 16-token pages run as one block-merge launch: in pages of 2, 8 or 24 tokens
    # it is read in place by the split-context kernel with its merge pass (another partition order, so compared
    # with the oracle, not bit for bit), the last page of every sequence partly filled.
    seq_lens = [1000] * 16
    q_lens = [1] * 16
    q, layouts = _same_tokens_two_page_sizes(500 + page_size, dtype, hq, hkv, d, seq_lens, q_lens, page_size)
    P, kp, vp, bt = layouts[0]
    out = M.paged_attention(torch.from_numpy(q).cuda(), torch.from_numpy(kp).cuda(), torch.from_numpy(vp).cuda(),
                            torch.from_numpy(bt).cuda(), torch.tensor(seq_lens, dtype=torch.int32).cuda(),
                            torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32).cuda(),
                            max_q_len=1, max_seq_len=1000, sum_seq_lens=int(sum(seq_lens)))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = O.paged_attention(q, kp, vp, bt, np.asarray(seq_lens, np.int32),
                            np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32), hq, hkv, d, P,
                            dtype=O.F16 if dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    say(f"[small pages {page_size}] {dtype} D={d}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= (2e-3 if dtype == "f16" else 1e-5)


@pytest.mark.parametrize("hints", [False, True])
@pytest.mark.parametrize("dtype,hq,hkv,d,page_size", [
    ("f16", 28, 4, 128, 4), ("f16", 28, 4, 128, 8), ("f16", 28, 4, 128, 12), ("f16", 28, 4, 128, 24),
    ("f16", 14, 2, 64, 8), ("f16", 14, 2, 64, 40), ("f32", 28, 4, 128, 2), ("f32", 28, 4, 128, 6),
    ("f32", 14, 2, 64, 4), ("f32", 14, 2, 64, 12)])
def test_prefill_token_pages_match_oracle_and_16_token_pages(dtype, hq, hkv, d, page_size, hints):
    # Page sizes that are not a multiple of 16 but a multiple of the tokens one 64-lane load of the prefill
    # kernel covers (F16 D=128: 4, D=64: 8; F32 D=128: 2, D=64: 4) run the prefill kernel in place, each load
    # with its own page: chunks with and without a cached prefix, a long context whose keys are split across
    # blocks and merged, and a decode row.  With host hints the decode row runs in a launch of its own (the
    # split-context kernel's token pages, whose partitions may differ from the 16-token plan's) beside the
    # prefill launch.  Every row within the bar of the oracle; the prefill kernel's rows (all of them without
    # hints) bit for bit the 16-token-page result.
    q_lens = [200, 64, 130, 1, 96]
    seq_lens = [700, 64, 130 + 5 * page_size + 3, 333, 96 + 6000 + page_size // 2]
    q, layouts = _same_tokens_two_page_sizes(800 + page_size + d, dtype, hq, hkv, d, seq_lens, q_lens, page_size)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    kw = dict(seq_lens_host=np.asarray(seq_lens, np.int32), cu_q_lens_host=cu) if hints else {}
    say(f"[prefill token pages {page_size}] {dtype} D={d} hints={hints}: q {q_lens} seq {seq_lens}")
    outs = []
    for P, kp, vp, bt in layouts:
        out = M.paged_attention(torch.from_numpy(q).cuda(), torch.from_numpy(kp).cuda(), torch.from_numpy(vp).cuda(),
                                torch.from_numpy(bt).cuda(), torch.tensor(seq_lens, dtype=torch.int32).cuda(),
                                torch.from_numpy(cu).cuda(), max_q_len=max(q_lens), max_seq_len=max(seq_lens),
                                sum_seq_lens=int(sum(seq_lens)), **kw)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    P, kp, vp, bt = layouts[0]
    ref = O.paged_attention(q, kp, vp, bt, np.asarray(seq_lens, np.int32), cu, hq, hkv, d, P,
                            dtype=O.F16 if dtype == "f16" else O.F32, num_threads=16)
    finite = bool(np.isfinite(outs[0]).all())
    err = float(np.abs(outs[0].astype(np.float64) - ref).max()) if finite else float("inf")
    view = np.uint16 if dtype == "f16" else np.uint32
    rows = np.ones(int(cu[-1]), bool)
    if hints:
        rows[cu[3]:cu[4]] = False  # the decode row's launch
    diff = int(np.count_nonzero(outs[0][:, rows].view(view) != outs[1][:, rows].view(view)))
    say(f"[prefill token pages {page_size}] {dtype} D={d} hints={hints}: max-abs vs oracle {err:.3e}; "
        f"{diff} prefill-kernel outputs differ from 16-token pages")
    assert finite and err <= (2e-3 if dtype == "f16" else 1e-5) and diff == 0


@pytest.mark.parametrize("page_size", [48, 80, 272])
@pytest.mark.parametrize("dtype,hq,hkv,d", [("f16", 28, 4, 128), ("f32", 14, 2, 64)])
def test_prefill_page_sizes_multiple_of_16_match_oracle_and_16_token_pages(page_size, dtype, hq, hkv, d):
    # Page sizes that are multiples of 16 but not powers of two run the chunked-prefill kernel in place (its
    # page arithmetic is a multiply and a shift): chunks with and without a cached prefix, a page boundary
    # inside most 8-token load runs' neighbourhoods, and a decode row; bit for bit the 16-token-page result.
    q_lens = [200, 64, 130, 1]
    seq_lens = [700, 64, 130 + 5 * page_size + 24, 333]
    q, layouts = _same_tokens_two_page_sizes(700 + page_size, dtype, hq, hkv, d, seq_lens, q_lens, page_size)
    outs = []
    for P, kp, vp, bt in layouts:
        out = M.paged_attention(torch.from_numpy(q).cuda(), torch.from_numpy(kp).cuda(), torch.from_numpy(vp).cuda(),
                                torch.from_numpy(bt).cuda(), torch.tensor(seq_lens, dtype=torch.int32).cuda(),
                                torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32).cuda(),
                                max_q_len=max(q_lens), max_seq_len=max(seq_lens), sum_seq_lens=int(sum(seq_lens)))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    P, kp, vp, bt = layouts[0]
    ref = O.paged_attention(q, kp, vp, bt, np.asarray(seq_lens, np.int32),
                            np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32), hq, hkv, d, P,
                            dtype=O.F16 if dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(outs[0].astype(np.float64) - ref).max())
    view = np.uint16 if dtype == "f16" else np.uint32
    diff = int(np.count_nonzero(outs[0].view(view) != outs[1].view(view)))
    say(f"[prefill page size {page_size}] {dtype} D={d}: max-abs vs oracle {err:.3e}; "
        f"{diff} outputs differ from 16-token pages")
    assert np.isfinite(outs[0]).all() and err <= (2e-3 if dtype == "f16" else 1e-5) and diff == 0


@pytest.mark.parametrize("page_size,seq_len,q_len", [(16, 8192, 1), (16, 1000, 1), (5, 700, 1), (16, 1000, 200)])
def test_pages_past_2_pow_31_elements(page_size, seq_len, q_len):
    # Page ids above 2^31 / (Hkv * page_size * D) put their elements past 2^31 in the pool, so every offset must
    # be 64-bit: the split-context kernel (1000 tokens, ragged pair), the block-merge launch (two uniform 8K
    # sequences: 4 partitions), the repack of odd page sizes and the prefill kernel (200-token chunks).  The
    # pools are ~4 GiB each on the device, with only the used pages written; the oracle sees a compact host copy
    # of those pages.
    hq, hkv, d, n = 32, 8, 128, 2
    stride = hkv * page_size * d
    first = (1 << 31) // stride + 7
    lens = [seq_len, seq_len if seq_len == 8192 else seq_len // 2 + 3]
    need = [math.ceil(L / page_size) for L in lens]
    rng = np.random.default_rng(17 + page_size + q_len)
    ids = first + rng.permutation(sum(need) + 3)[:sum(need)].astype(np.int64)
    num_pages = int(ids.max()) + 1
    assert int(ids.min()) * stride > (1 << 31)
    bt = np.zeros((n, max(need)), np.int32)
    bt[0, :need[0]] = ids[:need[0]]
    bt[1, :need[1]] = ids[need[0]:]
    kp = torch.empty((num_pages, 1, hkv, page_size, d), dtype=torch.float16, device="cuda")
    vp = torch.empty_like(kp)
    used = torch.from_numpy(ids).cuda()
    g = torch.Generator(device="cuda").manual_seed(5)
    kvals = (torch.randn((len(ids), 1, hkv, page_size, d), generator=g, device="cuda") * 0.3).half()
    vvals = (torch.randn((len(ids), 1, hkv, page_size, d), generator=g, device="cuda") * 0.3).half()
    kp[used] = kvals
    vp[used] = vvals
    cu = np.array([0, q_len, 2 * q_len], np.int32)
    q = (torch.randn((hq, n * q_len, d), generator=g, device="cuda") * 0.3).half()
    out = M.paged_attention(q, kp, vp, torch.from_numpy(bt).cuda(), torch.tensor(lens, dtype=torch.int32).cuda(),
                            torch.from_numpy(cu).cuda(), max_q_len=q_len, max_seq_len=max(lens),
                            sum_seq_lens=int(sum(lens)))
    torch.cuda.synchronize()
    # Oracle on a compact pool: page ids[i] -> i.
    remap = {int(v): i for i, v in enumerate(ids)}
    bt_c = np.vectorize(lambda x: remap.get(int(x), 0))(bt).astype(np.int32)
    ref = O.paged_attention(q.cpu().numpy(), kvals.cpu().numpy(), vvals.cpu().numpy(), bt_c,
                            np.asarray(lens, np.int32), cu, hq, hkv, d, page_size, dtype=O.F16, num_threads=16)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    say(f"[2^31] page size {page_size}, lengths {lens}, q_len {q_len}: pool {num_pages} pages, "
        f"max-abs vs oracle {err:.3e}")
    del kp, vp
    torch.cuda.empty_cache()
    assert err <= 2e-3
