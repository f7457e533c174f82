"""GPU parity of the fused RoPE + KV-append kernel (mvr_rope_append) against the oracle.

The rotation is a fixed sequence of rounded multiplies and adds per element
and the append is a copy, so the bar is bit-exact: rotated queries, rotated
keys in their page slots and copied values equal the oracle's
(oracle/kv_append_oracle.c) bit for bit, and every slot the append does not
own keeps its previous contents.  Covers F16 and F32, Neox and Interleaved
rotation, head_dim 64/128, page sizes 16 and 5, ragged batches crossing page
boundaries (5 requests, and 63/64/65 around the request lookup's wavefront
boundary), in-place and token-major layouts, the reference's paged-cache
unit tests (paged_cache.rs:560-1017) replayed through the kernel, the
attention call that follows, and a full-size Llama-3-8B decode step.
"""
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

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kv_append_kats.json")))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()
    O.build()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


def make_case(seed, dtype, hq, hkv, d, page_size, cached, q_lens, num_pages=96, rope_len=None):
    rng = np.random.default_rng(seed)
    npd = np.float16 if dtype == "f16" else np.float32
    cached = np.asarray(cached, np.int32)
    q_lens = np.asarray(q_lens, np.int32)
    seq_lens = (cached + q_lens).astype(np.int32)
    need = [math.ceil(int(L) / page_size) for L in seq_lens]
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(need), max(need)), np.int32)
    used = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[used:used + n]
        used += n
    assert used <= num_pages
    T = int(q_lens.sum())
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    rope_len = rope_len or int(seq_lens.max()) + 3
    cos, sin = W.rope_tables(d, 10000.0, rope_len, npd)
    return dict(
        dtype=dtype, npd=npd, bt=bt, seq_lens=seq_lens, cu=cu, cos=cos, sin=sin,
        q=(rng.standard_normal((hq, T, d)) * 2).astype(npd),
        k=(rng.standard_normal((hkv, T, d)) * 2).astype(npd),
        v=(rng.standard_normal((hkv, T, d)) * 2).astype(npd),
        kp=rng.standard_normal((num_pages, 1, hkv, page_size, d)).astype(npd),
        vp=rng.standard_normal((num_pages, 1, hkv, page_size, d)).astype(npd))


def run_oracle(c, rope_type):
    kp, vp = c["kp"].copy(), c["vp"].copy()
    q_out = O.rope_append(c["q"], c["k"], c["v"], c["cos"], c["sin"], c["bt"], c["seq_lens"], c["cu"], kp, vp,
                          rope_type, O.F16 if c["dtype"] == "f16" else O.F32)
    return q_out, kp, vp


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_hip(c, rope_type, in_place=False, token_major=False):
    q = dev(c["q"])
    k, v = dev(c["k"]), dev(c["v"])
    if token_major:  # [T, H, D] storage viewed as [H, T, D]
        q = q.transpose(0, 1).contiguous().transpose(0, 1)
        k = k.transpose(0, 1).contiguous().transpose(0, 1)
    kp, vp = dev(c["kp"]), dev(c["vp"])
    single = len(c["seq_lens"]) == 1
    q_out = M.rope_append(q, k, v, dev(c["cos"]), dev(c["sin"]), dev(c["bt"]),
                          None if single else dev(c["seq_lens"]), None if single else dev(c["cu"]), kp, vp,
                          q_out=q if in_place else None, max_seq_len=int(c["seq_lens"].max()), rope_type=rope_type)
    torch.cuda.synchronize()
    return q_out.cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy()


def assert_same(got, want):
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("rope_type", [M.ROPE_NEOX, M.ROPE_INTERLEAVED])
@pytest.mark.parametrize("d", [64, 128])
def test_ragged_batch_is_bit_exact(dtype, rope_type, d):
    say(f"[rope-append] ragged batch {dtype} rope={rope_type} D={d}")
    c = make_case(11 + d + rope_type, dtype, 8, 2, d, 16, cached=[0, 37, 128, 5, 300], q_lens=[1, 16, 3, 40, 17])
    q_ref, kp_ref, vp_ref = run_oracle(c, rope_type)
    q_out, kp, vp = run_hip(c, rope_type)
    assert_same(q_out, q_ref)
    assert_same(kp, kp_ref)
    assert_same(vp, vp_ref)
    assert not np.array_equal(bits(kp), bits(c["kp"]))  # something was written


@pytest.mark.parametrize("n", [63, 64, 65])
def test_request_lookup_at_the_wavefront_boundary(n):
    """The kernel finds a token's request with one wavefront-wide ballot over cu_q_lens for up to 63
    requests and by binary search beyond; batches of 63, 64 and 65 ragged requests (1..4 new tokens on
    0..40 cached ones) take both paths and their boundary."""
    say(f"[rope-append] {n} requests")
    rng = np.random.default_rng(n)
    cached = [int(x) for x in rng.integers(0, 41, size=n)]
    q_lens = [int(x) for x in rng.integers(1, 5, size=n)]
    c = make_case(90 + n, "f16", 8, 2, 64, 16, cached=cached, q_lens=q_lens, num_pages=256)
    q_ref, kp_ref, vp_ref = run_oracle(c, M.ROPE_NEOX)
    q_out, kp, vp = run_hip(c, M.ROPE_NEOX)
    assert_same(q_out, q_ref)
    assert_same(kp, kp_ref)
    assert_same(vp, vp_ref)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_odd_page_size_in_place_and_token_major(dtype):
    say(f"[rope-append] page size 5, in place, token-major {dtype}")
    c = make_case(5, dtype, 12, 4, 64, 5, cached=[3, 0, 11], q_lens=[9, 5, 1], num_pages=40)
    q_ref, kp_ref, vp_ref = run_oracle(c, M.ROPE_NEOX)
    for in_place, token_major in [(True, False), (False, True)]:
        q_out, kp, vp = run_hip(c, M.ROPE_NEOX, in_place=in_place, token_major=token_major)
        assert_same(q_out, q_ref)
        assert_same(kp, kp_ref)
        assert_same(vp, vp_ref)


def test_single_request_without_length_tables():
    say("[rope-append] single request, no seq_lens / cu_q_lens")
    c = make_case(6, "f16", 32, 8, 128, 16, cached=[1000], q_lens=[37], num_pages=80)
    q_ref, kp_ref, vp_ref = run_oracle(c, M.ROPE_INTERLEAVED)
    q_out, kp, vp = run_hip(c, M.ROPE_INTERLEAVED)
    assert_same(q_out, q_ref)
    assert_same(kp, kp_ref)
    assert_same(vp, vp_ref)


class GpuPagedCache:
    """The paged-cache bookkeeping of the reference's unit tests on host, with every append run by the kernel:
    F32, one KV head, head_dim 8, identity rotation (cos 1, sin 0), token value = position."""

    def __init__(self, page_size, capacity=16, seed=0):
        self.page_size = page_size
        rng = np.random.default_rng(seed)
        self.free = [int(p) for p in rng.permutation(capacity)]
        self.writable = np.zeros(capacity, np.uint8)
        self.table, self.cached = [], 0
        self.kp = torch.full((capacity, 1, 1, page_size, 8), -1.0, device="cuda")
        self.vp = torch.full((capacity, 1, 1, page_size, 8), -1.0, device="cuda")
        self.cos = torch.ones((64, 4), device="cuda")
        self.sin = torch.zeros((64, 4), device="cuda")

    def append(self, start, count, offset=100):
        assert start == self.cached
        need = -(-(start + count) // self.page_size)
        while len(self.table) < need:
            p = self.free.pop()
            self.writable[p] = 1
            self.table.append(p)
        pos = torch.arange(start, start + count, dtype=torch.float32, device="cuda")
        k = pos[None, :, None].expand(1, count, 8).contiguous()
        v = (pos + offset)[None, :, None].expand(1, count, 8).contiguous()
        q = torch.zeros((1, count, 8), device="cuda")
        bt = torch.tensor([self.table], dtype=torch.int32, device="cuda")
        a = M.make_rope_append_args(q, k, v, self.cos, self.sin, bt, None, None, self.kp, self.vp, q,
                                    max_seq_len=start + count)
        M.validate_rope_append(a, np.array([self.table], np.int32), None, None, self.writable)
        M.rope_append(q, k, v, self.cos, self.sin, bt, None, None, self.kp, self.vp, q_out=q,
                      max_seq_len=start + count)
        torch.cuda.synchronize()
        self.cached += count

    def truncate(self, n):
        keep = -(-n // self.page_size)
        for p in self.table[keep:]:
            self.writable[p] = 0
            self.free.append(p)
        self.table, self.cached = self.table[:keep], n

    def adopt_prefix_pages(self, k):
        for i in range(k):
            canonical = self.free.pop(0)
            self.kp[canonical] = self.kp[self.table[i]]
            self.vp[canonical] = self.vp[self.table[i]]
            self.writable[canonical] = 0
            self.writable[self.table[i]] = 0
            self.free.append(self.table[i])
            self.table[i] = canonical

    def gather(self, pool):
        ids = torch.tensor(self.table, dtype=torch.int32, device="cuda")
        out = M.reconstruct_contiguous(pool, ids, self.cached)
        torch.cuda.synchronize()
        rows = out[0, 0].cpu().numpy()
        assert (rows == rows[:, :1]).all()
        return [int(x) for x in rows[:, 0]]


@pytest.mark.parametrize("case", KATS["cases"], ids=[c["name"] for c in KATS["cases"]])
def test_reference_append_cases_through_the_kernel(case):
    say(f"[rope-append] reference case {case['name']}")
    m = GpuPagedCache(case["page_size"], seed=1)
    for op in case["ops"]:
        getattr(m, op[0])(*op[1:])
    assert len(m.table) == case["expected_pages"]
    assert m.gather(m.kp) == case["expected_key"]
    assert m.gather(m.vp) == case["expected_value"]


def test_append_then_attention_matches_the_oracle_pipeline():
    """forward_attention's order: RoPE + append, then attention over the grown cache."""
    say("[rope-append] append then attention (decode + verify rows)")
    c = make_case(7, "f16", 32, 8, 128, 16, cached=[500, 1023, 64, 2047], q_lens=[1, 5, 1, 5], num_pages=320)
    # Values N(0,1)*0.3 as in the workloads, so outputs stay below 1 and 2e-3 is a real bar (one f16 ulp is 2e-3
    # at 2..4 and 7.8e-3 at 8..16).
    for name, scale in (("kp", 0.3), ("vp", 0.3), ("q", 0.15), ("k", 0.15), ("v", 0.15)):
        c[name] = (c[name] * np.float16(scale)).astype(np.float16)
    q_ref, kp_ref, vp_ref = run_oracle(c, M.ROPE_NEOX)
    att_ref = O.paged_attention(q_ref, kp_ref, vp_ref, c["bt"], c["seq_lens"], c["cu"], 32, 8, 128, 16, dtype=O.F16)
    q = dev(c["q"])
    kp, vp = dev(c["kp"]), dev(c["vp"])
    bt, sl, cu = dev(c["bt"]), dev(c["seq_lens"]), dev(c["cu"])
    M.rope_append(q, dev(c["k"]), dev(c["v"]), dev(c["cos"]), dev(c["sin"]), bt, sl, cu, kp, vp, q_out=q,
                  max_seq_len=int(c["seq_lens"].max()))
    out = M.paged_attention(q, kp, vp, bt, sl, cu, max_q_len=5, max_seq_len=int(c["seq_lens"].max()))
    torch.cuda.synchronize()
    assert_same(q.cpu().numpy(), q_ref)
    err = np.abs(out.float().cpu().numpy() - att_ref).max()
    say(f"[rope-append] attention after append: max-abs {err:.3e}")
    assert err <= 2e-3


def test_full_size_decode_step_writes_only_its_slots():
    """Llama-3-8B decode, batch 64 at position 8191 of 8192, pools of 32768 pages (1 GiB each): the new rows
    equal the oracle's rotation bit for bit and every other slot of both pools is unchanged."""
    say("[rope-append] full-size decode step, 64 x 8192")
    w = W.llama3_8b_decode_b64_8k_f16()
    rng = np.random.default_rng(8)
    B, hq, hkv, d, P = w.num_seqs, w.num_q_heads, w.num_kv_heads, w.head_dim, w.page_size
    g = torch.Generator(device="cuda").manual_seed(8)
    kp = torch.randn((w.num_pages, 1, hkv, P, d), generator=g, device="cuda").half()
    vp = torch.randn((w.num_pages, 1, hkv, P, d), generator=g, device="cuda").half()
    kp0, vp0 = kp.clone(), vp.clone()
    q = rng.standard_normal((hq, B, d)).astype(np.float16)
    k = rng.standard_normal((hkv, B, d)).astype(np.float16)
    v = rng.standard_normal((hkv, B, d)).astype(np.float16)
    cos, sin = W.rope_tables(d, 500000.0, 8192, np.float16)
    bt, sl, cu = dev(w.block_tables), dev(w.seq_lens), dev(w.cu_q_lens)
    q_out = M.rope_append(dev(q), dev(k), dev(v), dev(cos), dev(sin), bt, sl, cu, kp, vp, max_seq_len=8192)
    torch.cuda.synchronize()
    pages = torch.from_numpy(w.block_tables[:, 8191 // P].astype(np.int64)).cuda()
    slot = 8191 % P
    # Every request's new token sits at position 8191: rotate each (head, request) row as its own q_len-1 row.
    rk = O.rope(k.reshape(hkv * B, 1, d), cos, sin, 8191, O.ROPE_NEOX, O.F16).reshape(hkv, B, d)
    rq = O.rope(q.reshape(hq * B, 1, d), cos, sin, 8191, O.ROPE_NEOX, O.F16).reshape(hq, B, d)
    np.testing.assert_array_equal(bits(kp[pages, 0, :, slot].cpu().numpy()), bits(rk.transpose(1, 0, 2)))
    np.testing.assert_array_equal(bits(vp[pages, 0, :, slot].cpu().numpy()), bits(v.transpose(1, 0, 2)))
    np.testing.assert_array_equal(bits(q_out.cpu().numpy()), bits(rq))
    mask = torch.ones((w.num_pages, P), dtype=torch.bool, device="cuda")
    mask[pages, slot] = False
    assert torch.equal(kp[:, 0].transpose(1, 2)[mask], kp0[:, 0].transpose(1, 2)[mask])
    assert torch.equal(vp[:, 0].transpose(1, 2)[mask], vp0[:, 0].transpose(1, 2)[mask])
