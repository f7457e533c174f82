"""Pins the oracle's RoPE + KV-append restatement (oracle/kv_append_oracle.c).

* page append: the reference's own paged-cache unit tests as golden vectors
  (tests/golden/kv_append_kats.json, paged_cache.rs:560-1017), its read-only
  and empty-append errors, and the multi-head slot layout;
* rotation: the textbook 2-D case (x = (1, 0) at position p -> (cos p, sin p)),
  the complex-number form of RoPE in float64, the relative-position property
  <R(m)q, R(n)k> = f(m - n), Neox == Interleaved after a fixed permutation of
  dims, and the per-operation rounding in F32 and F16 against numpy's own
  float32 / float16 arithmetic;
* the batched entry against the per-request composition.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
import workloads as W

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "kv_append_kats.json")))
POISON = 0xDEADBEEF


class PagedCacheModel:
    """The reference's page bookkeeping, reduced to what decides where an append writes: block table,
    cached_token_count, free list and PendingWrite state (paged_cache.rs:290-327, request_state.rs:106-178)."""

    def __init__(self, page_size, capacity=16, seed=0):
        self.page_size = page_size
        rng = np.random.default_rng(seed)
        self.free = [int(p) for p in rng.permutation(capacity)]
        self.writable = np.zeros(capacity, np.uint8)
        self.table = []
        self.cached = 0
        self.kpool = np.full((capacity, 1, 1, page_size, 1), POISON, np.uint32)
        self.vpool = np.full((capacity, 1, 1, page_size, 1), POISON, np.uint32)

    def allocate(self):
        p = self.free.pop()
        self.writable[p] = 1
        return p

    def append(self, start, count, offset=100):
        assert start == self.cached  # validate_cache_append (kv_cache/utils.rs:20-24)
        need = -(-(start + count) // self.page_size)
        while len(self.table) < need:
            self.table.append(self.allocate())
        key = np.arange(start, start + count, dtype=np.uint32).reshape(1, count, 1)
        value = np.arange(offset + start, offset + start + count, dtype=np.uint32).reshape(1, count, 1)
        O.append_pages(self.kpool, self.vpool, self.table, start, key, value, self.writable)
        self.cached += count

    def truncate(self, n):
        keep = -(-n // self.page_size)
        for p in self.table[keep:]:
            self.writable[p] = 0
            self.free.append(p)
        self.table = self.table[:keep]
        self.cached = n

    def adopt_prefix_pages(self, k):
        """Swap the first k pages for canonical read-only copies (record_prefix_publication)."""
        for i in range(k):
            canonical = self.free.pop(0)
            self.kpool[canonical] = self.kpool[self.table[i]]
            self.vpool[canonical] = self.vpool[self.table[i]]
            self.writable[canonical] = 0
            self.writable[self.table[i]] = 0
            self.free.append(self.table[i])
            self.table[i] = canonical

    def gather(self, pool):
        return [int(pool[self.table[t // self.page_size], 0, 0, t % self.page_size, 0]) for t in range(self.cached)]


@pytest.mark.parametrize("case", KATS["cases"], ids=[c["name"] for c in KATS["cases"]])
def test_reference_append_cases(case):
    for seed in range(3):
        m = PagedCacheModel(case["page_size"], seed=seed)
        for op in case["ops"]:
            getattr(m, op[0])(*op[1:])
        assert len(m.table) == case["expected_pages"]
        assert m.gather(m.kpool) == case["expected_key"]
        assert m.gather(m.vpool) == case["expected_value"]


def test_append_refuses_read_only_pages_and_empty_tensors():
    m = PagedCacheModel(2)
    m.append(0, 1)
    m.adopt_prefix_pages(1)
    with pytest.raises(O.OracleError) as e:
        m.append(1, 1)  # slot 1 of the adopted (written, shared) page
    assert str(e.value) == KATS["read_only_message"].format(m.table[0])
    assert e.value.code == O.APPEND_E_READ_ONLY
    with pytest.raises(O.OracleError) as e:
        O.append_pages(m.kpool, m.vpool, m.table, 1, np.zeros((1, 0, 1), np.uint32), np.zeros((1, 0, 1), np.uint32))
    assert str(e.value) == KATS["empty_message"]
    with pytest.raises(O.OracleError) as e:  # no page for position 2
        O.append_pages(m.kpool, m.vpool, m.table, 2, np.zeros((1, 1, 1), np.uint32), np.zeros((1, 1, 1), np.uint32))
    assert e.value.code == O.APPEND_E_MISSING


def test_append_multi_head_layout():
    """[Hkv, n, D] rows land at ((page*Hkv + h)*P + slot)*D (kv_cache/utils.rs:55-74)."""
    hkv, P, D, N = 3, 4, 5, 6
    kp = np.zeros((N, 1, hkv, P, D), np.float32)
    vp = np.zeros_like(kp)
    ids = [4, 1, 5]
    key = np.arange(hkv * 7 * D, dtype=np.float32).reshape(hkv, 7, D)
    O.append_pages(kp, vp, ids, 3, key, -key)
    for h in range(hkv):
        for t in range(7):
            pos = 3 + t
            np.testing.assert_array_equal(kp[ids[pos // P], 0, h, pos % P], key[h, t])
            np.testing.assert_array_equal(vp[ids[pos // P], 0, h, pos % P], -key[h, t])
    assert not kp[ids[0], 0, :, :3].any()


def _tables(d, n, dtype=np.float32, base=10000.0):
    c, s = W.rope_tables(d, base, n, dtype)
    return c, s


@pytest.mark.parametrize("rope_type", [O.ROPE_NEOX, O.ROPE_INTERLEAVED])
def test_rope_textbook_two_dims(rope_type):
    p = np.arange(9, dtype=np.float64)
    cos, sin = np.cos(p)[:, None], np.sin(p)[:, None]
    x = np.tile(np.array([1.0, 0.0]), (1, 9, 1))
    y = O.rope_f64(x, cos, sin, 0, rope_type)
    np.testing.assert_allclose(y[0, :, 0], np.cos(p), rtol=0, atol=1e-15)
    np.testing.assert_allclose(y[0, :, 1], np.sin(p), rtol=0, atol=1e-15)
    y32 = O.rope(x.astype(np.float32), cos.astype(np.float32), sin.astype(np.float32), 0, rope_type, O.F32)
    np.testing.assert_array_equal(y32[0, :, 0], np.cos(p).astype(np.float32))


def test_rope_is_complex_rotation_and_relative():
    rng = np.random.default_rng(1)
    d, L = 16, 40
    angle = np.arange(L)[:, None] * (1.0 / 10000.0 ** (np.arange(0, d, 2) / d))[None, :]
    c, s = np.cos(angle), np.sin(angle)  # exact float64 tables: cos^2 + sin^2 = 1 to 1 ulp
    x = rng.standard_normal((2, 5, d))
    y = O.rope_f64(x, c, s, 7, O.ROPE_NEOX)
    z = (x[..., :d // 2] + 1j * x[..., d // 2:]) * (c[7:12] + 1j * s[7:12])[None]
    np.testing.assert_allclose(y[..., :d // 2], z.real, atol=1e-13)
    np.testing.assert_allclose(y[..., d // 2:], z.imag, atol=1e-13)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-13)
    # <R(m) q, R(n) k> depends on m - n only.
    q, k = rng.standard_normal((1, 1, d)), rng.standard_normal((1, 1, d))
    dots = []
    for m, n in [(3, 1), (10, 8), (30, 28)]:
        dots.append(float((O.rope_f64(q, c, s, m) * O.rope_f64(k, c, s, n)).sum()))
    np.testing.assert_allclose(dots, dots[0], rtol=1e-12)
    assert abs(float((O.rope_f64(q, c, s, 3) * O.rope_f64(k, c, s, 0)).sum()) - dots[0]) > 1e-6


def test_interleaved_is_neox_on_permuted_dims():
    rng = np.random.default_rng(2)
    d, L = 64, 20
    for dtype, npd in [(O.F32, np.float32), (O.F16, np.float16)]:
        c, s = _tables(d, L, npd)
        x = (rng.standard_normal((3, 6, d)) * 0.7).astype(npd)
        perm = np.concatenate([np.arange(0, d, 2), np.arange(1, d, 2)])  # (2i, 2i+1) -> (i, i + D/2)
        yi = O.rope(x, c, s, 4, O.ROPE_INTERLEAVED, dtype)
        yn = O.rope(x[..., perm], c, s, 4, O.ROPE_NEOX, dtype)
        np.testing.assert_array_equal(yi[..., perm], yn)


@pytest.mark.parametrize("dtype,npd", [(O.F32, np.float32), (O.F16, np.float16)])
def test_rope_rounds_every_operation_in_the_activation_dtype(dtype, npd):
    rng = np.random.default_rng(3)
    d, L = 128, 64
    c, s = _tables(d, L, npd)
    x = (rng.standard_normal((4, 9, d)) * 3).astype(npd)
    y = O.rope(x, c, s, 50, O.ROPE_NEOX, dtype)
    h = d // 2
    cc, ss = c[50:59][None], s[50:59][None]
    a, b = x[..., :h], x[..., h:]
    with np.errstate(over="ignore"):
        ya = a * cc - b * ss  # numpy: each op in npd, rounded to nearest even
        yb = a * ss + b * cc
    np.testing.assert_array_equal(y[..., :h], ya)
    np.testing.assert_array_equal(y[..., h:], yb)
    if dtype == O.F16:
        # Not the same as rounding the exact result once: the intermediate roundings are real.
        exact = O.rope_f64(x.astype(np.float64), c.astype(np.float64), s.astype(np.float64), 50)
        assert (exact.astype(np.float16) != y).any()


def test_rope_position_offsets_follow_the_table_rows():
    rng = np.random.default_rng(4)
    d = 64
    c, s = _tables(d, 100, np.float16)
    x = rng.standard_normal((2, 5, d)).astype(np.float16)
    y = O.rope(x, c, s, 37, O.ROPE_NEOX, O.F16)
    for t in range(5):
        np.testing.assert_array_equal(y[:, t:t + 1], O.rope(x[:, t:t + 1], c, s, 37 + t, O.ROPE_NEOX, O.F16))
    with pytest.raises(O.OracleError):
        O.rope(x, c, s, 96, O.ROPE_NEOX, O.F16)  # rows 96..100 do not exist


@pytest.mark.parametrize("rope_type", [O.ROPE_NEOX, O.ROPE_INTERLEAVED])
def test_batched_rope_append_is_the_per_request_composition(rope_type):
    rng = np.random.default_rng(5)
    hq, hkv, d, P, N = 6, 2, 64, 16, 64
    q_lens = np.array([1, 17, 5], np.int32)
    cached = np.array([40, 0, 31], np.int32)
    seq_lens = cached + q_lens
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    T = int(cu[-1])
    perm = rng.permutation(N).astype(np.int32)
    bt = perm[:3 * 8].reshape(3, 8).copy()
    c, s = _tables(d, 128, np.float16)
    q = rng.standard_normal((hq, T, d)).astype(np.float16)
    k = rng.standard_normal((hkv, T, d)).astype(np.float16)
    v = rng.standard_normal((hkv, T, d)).astype(np.float16)
    kp = rng.standard_normal((N, 1, hkv, P, d)).astype(np.float16)
    vp = rng.standard_normal((N, 1, hkv, P, d)).astype(np.float16)
    kp2, vp2 = kp.copy(), vp.copy()
    q_out = O.rope_append(q, k, v, c, s, bt, seq_lens, cu, kp, vp, rope_type, O.F16)
    for b in range(3):
        sl = slice(cu[b], cu[b + 1])
        np.testing.assert_array_equal(q_out[:, sl], O.rope(q[:, sl], c, s, int(cached[b]), rope_type, O.F16))
        rk = O.rope(k[:, sl], c, s, int(cached[b]), rope_type, O.F16)
        n_pages = -(-int(seq_lens[b]) // P)
        O.append_pages(kp2, vp2, bt[b, :n_pages], int(cached[b]), rk, v[:, sl])
    np.testing.assert_array_equal(kp, kp2)
    np.testing.assert_array_equal(vp, vp2)
