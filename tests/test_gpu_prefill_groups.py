"""GPU parity of the prefill kernel's two block shapes at head_dim 64 and 128.

Up to D=128 a prefill block holds 128 grouped rows either in two groups of 4 wavefronts that take alternating
key tiles and merge at the end (two wavefronts per SIMD behind one barrier), or in one group of 4 wavefronts that
steps through every key tile (two such blocks per CU).  The planner takes one group for F16 grids of at least 4
blocks per CU and two otherwise; MVR_ATTN_PREFILL_GROUPS forces either (read once per process, so each shape runs
in a child process).  Both must meet the same bar against the oracle: 2e-3 (F16) / 1e-5 (F32).  Cases: the
Qwen2-7B chunk in F16 and F32, ragged chunks on long contexts at D=64 (key splits and their merge), a mixed
decode + prefill batch with host hints (the prefill launch of two), and the chunk and the mixed batch in pages of
8 (F16) and 2 (F32) tokens, which the prefill kernel reads in place; and, in this process, a batch whose grid
(48 sequences x 16 KV heads x 2 row tiles) takes one group by the planner's own rule.
"""
import os
import subprocess
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


def _ragged_chunks_d64():
    """Four chunks of 40..200 tokens on 3,000..7,000 cached tokens, 14/2 heads, D=64, F16: few blocks, so the keys
    are split and merged."""
    rng = np.random.default_rng(31)
    q = np.array([40, 200, 97, 130], np.int32)
    seq = (np.array([3000, 7000, 4100, 5555], np.int32) + q).astype(np.int32)
    pages = int(sum((int(L) + 15) // 16 for L in seq)) + 4
    bt = W._assign_pages(rng, seq, 16, pages)
    return W.Workload("ragged chunks d64", "f16", 14, 2, 64, 16, pages, 0.3, seq, q, bt, 31)


CASES = {
    "qwen2-7b-chunk-f16": (lambda: W.qwen2_7b_chunked_prefill_f16(), False),
    "qwen2-7b-chunk-f32": (lambda: W.qwen2_7b_chunked_prefill_f16("f32"), False),
    "ragged-chunks-d64": (_ragged_chunks_d64, False),
    "mixed-with-hints": (lambda: W.llama3_8b_mixed_decode_prefill_f16(num_decode=15, decode_ctx=2048), True),
    # pages of 8 and 2 tokens, read in place (token pages)
    "qwen2-7b-chunk-f16-p8": (lambda: W.repaged(W.qwen2_7b_chunked_prefill_f16(), 8), False),
    "qwen2-7b-chunk-f32-p2": (lambda: W.repaged(W.qwen2_7b_chunked_prefill_f16("f32"), 2), False),
    "mixed-with-hints-p8": (lambda: W.repaged(W.llama3_8b_mixed_decode_prefill_f16(num_decode=15, decode_ctx=2048), 8),
                            True),
}


def _attend(name):
    build, hints = CASES[name]
    w = build()
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    kw = dict(seq_lens_host=w.seq_lens, cu_q_lens_host=w.cu_q_lens) if hints else {}
    out = torch.full((w.num_q_heads, w.total_q, w.head_dim), float("nan"), dtype=t["q"].dtype, device="cuda")
    M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out,
                      max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()), **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _groups_child(name, path):
    """Child-process side: the case under the block shape the parent chose."""
    M.load_library()
    np.save(path, _attend(name))


_CHILD = (
    "import sys\n"
    "sys.path[:0] = sys.argv[3].split('|')\n"
    "import test_gpu_prefill_groups as T\n"
    "T._groups_child(sys.argv[1], sys.argv[2])\n"
    "print('groups done', flush=True)\n"
)


def _run_child(name, dst, groups):
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = "|".join([here, root, os.path.join(root, "oracle"), os.path.join(root, "mini-vllm-rs_amd")])
    child = subprocess.run([sys.executable, "-c", _CHILD, name, dst, paths],
                           env=dict(os.environ, MVR_ATTN_PREFILL_GROUPS=str(groups)), capture_output=True, text=True,
                           timeout=180)
    assert child.returncode == 0, child.stdout[-2000:] + child.stderr[-2000:]
    return np.load(dst)


@pytest.mark.parametrize("groups", [1, 2])
@pytest.mark.parametrize("name", list(CASES))
def test_prefill_block_shape_matches_oracle(name, groups, tmp_path):
    say(f"[prefill groups] {name}: {groups} group(s) per block (child process)")
    got = _run_child(name, str(tmp_path / f"g{groups}.npy"), groups)
    w = CASES[name][0]()
    q, k, v = W.host_values(w)
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    finite = bool(np.isfinite(got).all())
    err = float(np.abs(got - ref).max()) if finite else float("inf")
    say(f"[prefill groups] {name}: {groups} group(s): max-abs vs oracle {err:.3e}")
    assert finite and err <= TOL[w.dtype], err


def test_many_block_grid_takes_one_group_by_default():
    # 48 chunks of 130 tokens on 100 cached, 16/16 heads, D=128, F16: 1,536 blocks, 6 per CU.
    rng = np.random.default_rng(37)
    q = np.full(48, 130, np.int32)
    seq = (q + 100).astype(np.int32)
    pages = int(sum((int(L) + 15) // 16 for L in seq)) + 4
    bt = W._assign_pages(rng, seq, 16, pages)
    w = W.Workload("many blocks", "f16", 16, 16, 128, 16, pages, 0.3, seq, q, bt, 37)
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    out = torch.full((w.num_q_heads, w.total_q, w.head_dim), float("nan"), dtype=t["q"].dtype, device="cuda")
    M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], out,
                      max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = O.paged_attention(vals[0], vals[1], vals[2], w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads,
                            w.num_kv_heads, w.head_dim, w.page_size, dtype=O.F16, num_threads=16)
    finite = bool(np.isfinite(got).all())
    err = float(np.abs(got - ref).max()) if finite else float("inf")
    say(f"[prefill groups] 1,536-block grid (one group by default): max-abs vs oracle {err:.3e}")
    assert finite and err <= TOL["f16"], err
