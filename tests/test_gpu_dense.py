"""GPU parity of the dense layout of ragged batches.

A ragged batch of many sequences, most of whose slot == partition grid would
hold no work, numbers its live (sequence, partition) units densely from 0 and
lets each wavefront find its unit with a wave-wide scan of the sequence
lengths (dense_unit).  Same bar as every call: 2e-3 (F16) / 1e-5 (F32)
against the oracle.  Covers 64 sequences of 257..2049 tokens (F16, D=128), 150
sequences of 17..1024 tokens (more than one 64-sequence block of the scan, the
F16 D=64 kernel), 40 F32 sequences at D=64 and at D=128 (whose key rows
of 512 bytes take the finer dense split), and two such batches in pages of
8 and 5 tokens read in place (token pages), of which the first takes the
dense layout (from 8 tokens per page) and the second slot == partition.
By default a dense plan also splits
contexts into more partitions than the slot == partition plan of the same
batch (a higher fill target), which changes the rounding.  With the same
partitions the dense layout only changes which wavefront computes which
partition, so two child processes run the batch at a fixed number of chunks
per partition (MVR_ATTN_CHUNKS_PER_PARTITION, which also skips the re-split),
one with the dense layout and one with MVR_ATTN_DENSE_RAGGED=false, and the
results are compared bit for bit.  (The flags are read once per process; at
8 and 4 chunks per partition these batches take the dense layout by the
planner's rule: at least 32 sequences, estimated live fraction of the slot
grid below 0.7.)
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


def ragged_workload(name, dtype, hq, hkv, d, n, lo, hi, seed, page=16):
    rng = np.random.default_rng(seed)
    seq_lens = rng.integers(lo, hi, size=n, endpoint=True).astype(np.int32)
    pages = int(sum((int(L) + page - 1) // page for L in seq_lens)) + 8
    bt = W._assign_pages(rng, seq_lens, page, pages)
    return W.Workload(name, dtype, hq, hkv, d, page, pages, 0.3, seq_lens, np.ones(n, np.int32), bt, seed)


CASES = {
    "f16-d128-64x[257,2049]": ("f16", 32, 8, 128, 64, 257, 2049, 71),
    "f16-d64-150x[17,1024]": ("f16", 14, 2, 64, 150, 17, 1024, 72),
    "f32-d64-40x[100,3000]": ("f32", 14, 2, 64, 40, 100, 3000, 73),
    "f32-d128-40x[512,4096]": ("f32", 32, 8, 128, 40, 512, 4096, 74),
    # pages of 8 and 5 tokens, read in place (token pages): the dense layout from 8 tokens per page, the
    # slot == partition layout below
    "f16-d128-64x[257,2049]-p8": ("f16", 32, 8, 128, 64, 257, 2049, 75, 8),
    "f32-d64-40x[100,3000]-p5": ("f32", 14, 2, 64, 40, 100, 3000, 76, 5),
}


def _case(name):
    return ragged_workload(name, *CASES[name])


def _attend(w, vals=None):
    t = W.device_tensors(w, vals if vals is not None else W.host_values(w))
    args = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                       t["q"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    need = M.workspace_size(args)
    out = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                            max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    return out.cpu().numpy(), need


@pytest.mark.parametrize("name", list(CASES))
def test_dense_matches_oracle(name):
    w = _case(name)
    vals = W.host_values(w)
    got, _ = _attend(w, vals)
    q, k, v = vals
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    say(f"[dense] {name}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[w.dtype], err


def _layout_child(name, path):
    """Child-process side: the batch under the environment the parent chose."""
    M.load_library()
    out, need = _attend(_case(name))
    np.save(path, out)
    np.save(path + ".ws.npy", np.array([need], np.int64))


_CHILD = (
    "import sys\n"
    "sys.path[:0] = sys.argv[3].split('|')\n"
    "import test_gpu_dense as T\n"
    "T._layout_child(sys.argv[1], sys.argv[2])\n"
    "print('layout done', flush=True)\n"
)


FIXED_CHUNKS = {"f16-d128-64x[257,2049]": "8", "f16-d64-150x[17,1024]": "4", "f32-d128-40x[512,4096]": "8",
                "f16-d128-64x[257,2049]-p8": "8"}


def _run_child(name, dst, **env):
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = "|".join([here, root, os.path.join(root, "oracle"), os.path.join(root, "mini-vllm-rs_amd")])
    child = subprocess.run([sys.executable, "-c", _CHILD, name, dst, paths], env=dict(os.environ, **env),
                           capture_output=True, text=True, timeout=180)
    assert child.returncode == 0, child.stdout[-2000:] + child.stderr[-2000:]
    return np.load(dst), int(np.load(dst + ".ws.npy")[0])


@pytest.mark.parametrize("name", list(FIXED_CHUNKS))
def test_dense_bit_identical_to_slot_layout(name, tmp_path):
    cpp = FIXED_CHUNKS[name]
    say(f"[dense] {name}: dense and slot == partition layouts at {cpp} chunks per partition (child processes)")
    got, need = _run_child(name, str(tmp_path / "dense.npy"), MVR_ATTN_CHUNKS_PER_PARTITION=cpp)
    ref, ref_ws = _run_child(name, str(tmp_path / "slot.npy"), MVR_ATTN_CHUNKS_PER_PARTITION=cpp,
                             MVR_ATTN_DENSE_RAGGED="false")
    # Both layouts hold the same partitions, so the same workspace.
    assert need == ref_ws, (need, ref_ws)
    view = np.uint16 if got.dtype == np.float16 else np.uint32
    diff = int(np.count_nonzero(got.view(view) != ref.view(view)))
    say(f"[dense] {name}: {diff} of {got.size} outputs differ from the slot == partition layout "
        f"(workspace {need} vs {ref_ws} bytes)")
    assert diff == 0
