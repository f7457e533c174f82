"""Writes reference_kats.json: the closed-form attention cases of mini-vllm-rs's
own unit tests (src/models/backends/common.rs:1031-1203), as data.

Inputs and expected outputs are the values those tests state.  The paged
fixture (common.rs:1143-1203) asserts paged == contiguous attention and states
no numbers, so its expected output is evaluated here with textbook softmax
attention in numpy float64 (no oracle code involved).
Run: python tests/golden/make_golden.py
"""
import json
import os

import numpy as np


def textbook_attention(q, k, v, cached_kv_len):
    """q [Hq,q,D], k/v [Hkv,L,D] -> [Hq,q,D]; key j visible to query i iff j <= cached_kv_len + i."""
    hq, qlen, d = q.shape
    hkv = k.shape[0]
    rep = hq // hkv
    out = np.zeros_like(q, dtype=np.float64)
    for h in range(hq):
        kh, vh = k[h // rep], v[h // rep]
        s = q[h] @ kh.T / np.sqrt(d)
        for i in range(qlen):
            s[i, cached_kv_len + i + 1:] = -np.inf
        w = np.exp(s - s.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        out[h] = w @ vh
    return out


def main():
    cases = []
    # common.rs:1031-1047  contiguous_attention_computes_multi_head_attention
    cases.append(dict(name="contiguous_attention_computes_multi_head_attention", source="common.rs:1031-1047",
                      dtype="f32", num_q_heads=2, num_kv_heads=2, head_dim=1, cached_kv_len=1, q_len=1,
                      q=[0., 0.], k=[1., 2., 3., 4.], v=[2., 4., 10., 14.], expected=[3., 12.]))
    # common.rs:1049-1075  grouped_query_matmul_matches_repeated_kv_attention
    cases.append(dict(name="grouped_query_matmul_matches_repeated_kv_attention", source="common.rs:1049-1075",
                      dtype="f32", num_q_heads=4, num_kv_heads=1, head_dim=1, cached_kv_len=1, q_len=1,
                      q=[0., 0., 0., 0.], k=[1., 2.], v=[2., 6.], expected=[4., 4., 4., 4.]))
    # common.rs:1077-1093  contiguous_attention_applies_a_causal_prefill_mask
    cases.append(dict(name="contiguous_attention_applies_a_causal_prefill_mask", source="common.rs:1077-1093",
                      dtype="f32", num_q_heads=1, num_kv_heads=1, head_dim=1, cached_kv_len=0, q_len=3,
                      q=[0., 0., 0.], k=[1., 2., 3.], v=[1., 3., 5.], expected=[1., 2., 3.]))
    # common.rs:1095-1123  f16_rotary_frequencies_and_attention_preserve_dtype (attention half)
    cases.append(dict(name="f16_attention_preserves_dtype", source="common.rs:1095-1123",
                      dtype="f16", num_q_heads=1, num_kv_heads=1, head_dim=1, cached_kv_len=0, q_len=3,
                      q=[0., 0., 0.], k=[1., 2., 3.], v=[1., 3., 5.], expected=[1., 2., 3.]))
    # common.rs:1125-1141  contiguous_attention_decode_attends_to_the_cached_prefix
    cases.append(dict(name="contiguous_attention_decode_attends_to_the_cached_prefix", source="common.rs:1125-1141",
                      dtype="f32", num_q_heads=1, num_kv_heads=1, head_dim=1, cached_kv_len=3, q_len=1,
                      q=[0.], k=[1., 2., 3., 4.], v=[1., 3., 5., 7.], expected=[4.]))
    # common.rs:1143-1203  paged_attention_matches_contiguous_attention_across_partial_pages
    q = [0.2, -0.1, 0.4, 0.3, -0.2, 0.5, 0.1, -0.4]
    k_values = [0.1, 0.2, 0.3, -0.1, -0.2, 0.4, 0.5, 0.6, -0.3, 0.2]
    v_values = [1., 2., 3., 4., 5., 6., 7., 8., 9., 10.]
    key_pool = [0.5, 0.6, -0.3, 0.2, 99., 99., 88., 88., 88., 88., 88., 88., 0.1, 0.2, 0.3, -0.1, -0.2, 0.4]
    value_pool = [7., 8., 9., 10., 99., 99., 88., 88., 88., 88., 88., 88., 1., 2., 3., 4., 5., 6.]
    qa = np.array(q, dtype=np.float32).astype(np.float64).reshape(2, 2, 2)
    ka = np.array(k_values, dtype=np.float32).astype(np.float64).reshape(1, 5, 2)
    va = np.array(v_values, dtype=np.float32).astype(np.float64).reshape(1, 5, 2)
    expected = textbook_attention(qa, ka, va, cached_kv_len=3).reshape(-1).tolist()
    cases.append(dict(name="paged_attention_matches_contiguous_attention_across_partial_pages",
                      source="common.rs:1143-1203", dtype="f32", num_q_heads=2, num_kv_heads=1, head_dim=2,
                      cached_kv_len=3, q_len=2, q=q, k=k_values, v=v_values,
                      paged=dict(page_count=3, page_size=3, page_ids=[2, 0], cached_token_count=5,
                                 key_pool=key_pool, value_pool=value_pool),
                      expected=expected))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(path, "w") as f:
        json.dump(dict(tolerance=1e-5, tolerance_source="common.rs:984", cases=cases), f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
