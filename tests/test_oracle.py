"""Pins the oracle (CPU restatement of common.rs:739-978) before it is trusted.

Checks: the reference's own closed-form unit tests (golden fixture), its
paged == contiguous fixture with poisoned unused slots, f16 rounding against
numpy, an independent float64 evaluation against torch's SDPA, and
size-independent invariants chosen so that a dropped term, a wrong index or a
transposed operand fails.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")


def _kats():
    with open(GOLDEN) as f:
        return json.load(f)


def _dt(name):
    return O.F16 if name == "f16" else O.F32


@pytest.fixture(scope="module", autouse=True)
def _build_oracle():
    O.build()


@pytest.mark.parametrize("mode", [O.REF_CONCAT_V, O.REF_PAGEWISE_V, O.EXACT_F64])
def test_reference_unit_tests_contiguous(mode):
    kats = _kats()
    tol = kats["tolerance"]  # common.rs:984
    for case in kats["cases"]:
        hq, hkv, d = case["num_q_heads"], case["num_kv_heads"], case["head_dim"]
        c, ql = case["cached_kv_len"], case["q_len"]
        L = c + ql
        q = np.array(case["q"], np.float32).reshape(1, hq, ql, d)
        k = np.array(case["k"], np.float32).reshape(1, hkv, L, d)
        v = np.array(case["v"], np.float32).reshape(1, hkv, L, d)
        out = O.forward_contiguous_attention(q, k, v, hq, hkv, d, c, ql, dtype=_dt(case["dtype"]), mode=mode)
        np.testing.assert_allclose(out.reshape(-1), case["expected"], atol=tol, rtol=0, err_msg=case["name"])


@pytest.mark.parametrize("mode", [O.REF_CONCAT_V, O.REF_PAGEWISE_V, O.EXACT_F64])
def test_reference_paged_fixture_partial_pages(mode):
    """common.rs:1143-1203: block table [2, 0], partial last page, poison 99/88."""
    case = [c for c in _kats()["cases"] if "paged" in c][0]
    pg = case["paged"]
    kp = np.array(pg["key_pool"], np.float32).reshape(pg["page_count"], 1, 1, pg["page_size"], 2)
    vp = np.array(pg["value_pool"], np.float32).reshape(pg["page_count"], 1, 1, pg["page_size"], 2)
    q = np.array(case["q"], np.float32).reshape(1, 2, 2, 2)
    out = O.forward_paged_attention(q, kp, vp, pg["page_ids"], pg["page_size"], pg["cached_token_count"], 2, 1, 2,
                                    case["cached_kv_len"], case["q_len"], dtype=O.F32, mode=mode)
    np.testing.assert_allclose(out.reshape(-1), case["expected"], atol=1e-5, rtol=0)


def test_reference_error_paths():
    q = np.zeros((1, 1, 1, 1), np.float32)
    pool = np.zeros((2, 1, 1, 4, 1), np.float32)
    # common.rs:447-454: cached_token_count != cached_kv_len + q_len
    with pytest.raises(O.OracleError, match="reports sequence length 5, expected 4") as e:
        O.forward_paged_attention(q, pool, pool, [0, 1], 4, 5, 1, 1, 1, 3, 1)
    assert e.value.code == O.E_LENGTH
    # common.rs:776-781: pages do not cover the length
    with pytest.raises(O.OracleError, match="leaving 2 tokens uncovered") as e:
        O.forward_paged_attention(q, pool, pool, [1], 4, 6, 1, 1, 1, 5, 1)
    assert e.value.code == O.E_UNCOVERED
    with pytest.raises(O.OracleError) as e:
        O.forward_paged_attention(q, pool, pool, [7], 4, 2, 1, 1, 1, 1, 1)
    assert e.value.code == O.E_PAGE_ID


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, np.inf, -np.inf, 1.0 / 3.0], np.float32),
    ]).astype(np.float32)
    expected = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16_bits(float(x)) for x in vals], np.uint16)
    np.testing.assert_array_equal(got, expected)
    all_bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = ~np.isnan(all_bits.view(np.float16))
    back = np.array([O.f16_bits_to_f32(int(h)) for h in all_bits[finite]], np.float32)
    np.testing.assert_array_equal(back, all_bits[finite].view(np.float16).astype(np.float32))


def _random_case(rng, hq, hkv, d, page_size, page_count, seq_len, q_len, scale=0.5):
    pages_needed = math.ceil(seq_len / page_size)
    page_ids = rng.permutation(page_count)[:pages_needed]
    kp = (rng.standard_normal((page_count, 1, hkv, page_size, d)) * scale).astype(np.float32)
    vp = (rng.standard_normal((page_count, 1, hkv, page_size, d)) * scale).astype(np.float32)
    q = (rng.standard_normal((1, hq, q_len, d)) * scale).astype(np.float32)
    return q, kp, vp, page_ids


def _gather(pool, page_ids, L):
    """Contiguous [1, Hkv, L, D] from a pool (plain numpy indexing)."""
    parts = [pool[p, 0] for p in page_ids]
    return np.concatenate(parts, axis=1)[None, :, :L, :]


@pytest.mark.parametrize("hq,hkv,d,q_len,seq_len", [(14, 2, 64, 1, 37), (8, 2, 32, 5, 70), (4, 4, 16, 9, 9)])
def test_exact_f64_matches_torch_sdpa(hq, hkv, d, q_len, seq_len):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    q, kp, vp, ids = _random_case(rng, hq, hkv, d, 16, 12, seq_len, q_len)
    out = O.forward_paged_attention(q, kp, vp, ids, 16, seq_len, hq, hkv, d, seq_len - q_len, q_len,
                                    mode=O.EXACT_F64)
    k = torch.from_numpy(_gather(kp, ids, seq_len)).double().repeat_interleave(hq // hkv, dim=1)
    v = torch.from_numpy(_gather(vp, ids, seq_len)).double().repeat_interleave(hq // hkv, dim=1)
    qt = torch.from_numpy(q).double()
    c = seq_len - q_len
    mask = torch.arange(seq_len)[None, :] <= (c + torch.arange(q_len))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(qt, k, v, attn_mask=mask)
    np.testing.assert_allclose(out, ref[0].numpy(), atol=1e-12, rtol=0)


@pytest.mark.parametrize("dtype,tol", [(O.F32, 2e-6), (O.F16, 2e-3)])
def test_reference_dataflow_close_to_exact(dtype, tol):
    rng = np.random.default_rng(11)
    q, kp, vp, ids = _random_case(rng, 14, 2, 64, 16, 40, 500, 3)
    if dtype == O.F16:
        q, kp, vp = (x.astype(np.float16) for x in (q, kp, vp))
    ref = O.forward_paged_attention(q, kp, vp, ids, 16, 500, 14, 2, 64, 497, 3, dtype=dtype)
    exact = O.forward_paged_attention(q, kp, vp, ids, 16, 500, 14, 2, 64, 497, 3, dtype=dtype, mode=O.EXACT_F64)
    err = np.abs(ref - exact).max()
    assert err <= tol, err
    assert err > 0  # the dataflow mode does round: it is not the f64 path
    pagewise = O.forward_paged_attention(q, kp, vp, ids, 16, 500, 14, 2, 64, 497, 3, dtype=dtype,
                                         mode=O.REF_PAGEWISE_V)
    assert np.abs(pagewise - exact).max() <= tol


def test_invariant_block_table_permutation():
    """Moving pages to other physical slots (and the table with them) changes nothing, bit for bit."""
    rng = np.random.default_rng(3)
    q, kp, vp, ids = _random_case(rng, 8, 2, 32, 16, 20, 150, 2)
    perm = rng.permutation(20)
    kp2, vp2 = np.empty_like(kp), np.empty_like(vp)
    kp2[perm], vp2[perm] = kp, vp
    a = O.forward_paged_attention(q, kp, vp, ids, 16, 150, 8, 2, 32, 148, 2)
    b = O.forward_paged_attention(q, kp2, vp2, perm[ids], 16, 150, 8, 2, 32, 148, 2)
    np.testing.assert_array_equal(a, b)


def test_invariant_unused_slots_and_pages_ignored():
    """Poisoning every slot beyond the length and every page off the table changes nothing."""
    rng = np.random.default_rng(4)
    q, kp, vp, ids = _random_case(rng, 4, 1, 16, 16, 8, 35, 1)
    a = O.forward_paged_attention(q, kp, vp, ids, 16, 35, 4, 1, 16, 34, 1)
    kp2, vp2 = kp.copy(), vp.copy()
    unused = np.setdiff1d(np.arange(8), ids)
    kp2[unused], vp2[unused] = 1e4, -1e4
    kp2[ids[-1], :, :, 3:], vp2[ids[-1], :, :, 3:] = 99.0, 88.0  # 35 = 2*16 + 3 valid slots
    b = O.forward_paged_attention(q, kp2, vp2, ids, 16, 35, 4, 1, 16, 34, 1)
    np.testing.assert_array_equal(a, b)


def test_invariant_uniform_query_is_mean_of_visible_values():
    """q = 0 gives equal weights: output = mean of V over keys j <= c + i (closed form)."""
    rng = np.random.default_rng(5)
    _, kp, vp, ids = _random_case(rng, 6, 3, 8, 4, 10, 23, 4)
    q = np.zeros((1, 6, 4, 8), np.float32)
    out = O.forward_paged_attention(q, kp, vp, ids, 4, 23, 6, 3, 8, 19, 4, mode=O.EXACT_F64)
    v = _gather(vp, ids, 23)[0]
    for h in range(6):
        for i in range(4):
            np.testing.assert_allclose(out[h, i], v[h // 2, :20 + i].astype(np.float64).mean(axis=0), atol=1e-12)


def test_invariant_one_hot_key_selects_its_value():
    """A key aligned with a huge query wins the softmax: output is exactly that V row (GQA head mapping)."""
    rng = np.random.default_rng(6)
    hq, hkv, d, L = 4, 2, 8, 40
    _, kp, vp, ids = _random_case(rng, hq, hkv, d, 16, 6, L, 1, scale=0.01)
    q = np.zeros((1, hq, 1, d), np.float32)
    targets = {0: 5, 1: 17, 2: 33, 3: 39}
    for h, j in targets.items():
        kvh = h // (hq // hkv)
        vec = np.zeros(d, np.float32)
        vec[h] = 1.0
        kp[ids[j // 16], 0, kvh, j % 16] = vec * 30.0
        q[0, h, 0] = vec * 30.0
    out = O.forward_paged_attention(q, kp, vp, ids, 16, L, hq, hkv, d, L - 1, 1, mode=O.EXACT_F64)
    for h, j in targets.items():
        np.testing.assert_allclose(out[h, 0], vp[ids[j // 16], 0, h // 2, j % 16], atol=1e-9)


def test_batched_matches_request_level():
    rng = np.random.default_rng(8)
    hq, hkv, d, P, N = 8, 2, 32, 16, 64
    seq_lens, q_lens = [40, 16, 77], [1, 3, 5]
    kp = (rng.standard_normal((N, 1, hkv, P, d)) * 0.5).astype(np.float16)
    vp = (rng.standard_normal((N, 1, hkv, P, d)) * 0.5).astype(np.float16)
    perm = rng.permutation(N)
    bt = np.zeros((3, 8), np.int32)
    used = 0
    for s, L in enumerate(seq_lens):
        n = math.ceil(L / P)
        bt[s, :n] = perm[used:used + n]
        used += n
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = (rng.standard_normal((hq, int(cu[-1]), d)) * 0.5).astype(np.float16)
    out = O.paged_attention(q, kp, vp, bt, seq_lens, cu, hq, hkv, d, P, dtype=O.F16)
    for s, L in enumerate(seq_lens):
        ql = q_lens[s]
        rq = q[:, cu[s]:cu[s + 1]][None]
        ref = O.forward_paged_attention(rq, kp, vp, bt[s, :math.ceil(L / P)], P, L, hq, hkv, d, L - ql, ql,
                                        dtype=O.F16)
        np.testing.assert_array_equal(out[:, cu[s]:cu[s + 1]], ref)


def test_reconstruct_contiguous_is_exact_gather():
    rng = np.random.default_rng(9)
    pool = rng.standard_normal((9, 1, 2, 4, 3)).astype(np.float16)
    ids = [4, 0, 7]
    out = O.reconstruct_contiguous(pool, ids, 10, dtype=O.F16)
    np.testing.assert_array_equal(out, _gather(pool, ids, 10)[0])
