"""GPU parity of the split-context kernel's block shapes (wavefronts per block).

Plans without block merge run one unit (sequence, KV head, row tile,
partition) per wavefront, in blocks of 4 wavefronts or of 1 (the planner's
choice: 1 for dense plans, for F32, for ragged plans with a multiple of 32
units per sequence and for grids of fewer 4-wavefront blocks than CUs; 2 on
request).
The shape moves units between CUs and XCDs but changes nothing a unit
computes, so every shape must give the same bits.  Cases, one per branch:
  * 16 F16 sequences of 1,024..8,192 tokens, 32/8 heads, D=128 (slot layout,
    deep pipeline, 24 partitions: 192 units per sequence);
  * the same lengths in F32 (slot layout, two-chunk pipeline);
  * 48 F16 sequences of 512..4,096 tokens (dense layout);
  * one F32 sequence of 512 tokens, 14/2 heads, D=64 (32 units);
  * 24 F16 sequences of 5 query tokens on 1,024..4,096 cached tokens, 32/8
    heads (32-row tiles).
Each is checked against the oracle (2e-3 F16, 1e-5 F32) with the planner's
shape, and bit for bit against 1, 2 and 4 wavefronts per block forced by
MVR_ATTN_UNIT_WAVES in child processes (the flag is read once per process).
"""
import os
import subprocess
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (HERE, ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "mini-vllm-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

torch = pytest.importorskip("torch")
import mvr_attn as M  # noqa: E402
import oracle as O  # noqa: E402
import test_gpu_dense as D  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = {"f32": 1e-5, "f16": 2e-3}


def _verify_like(name, n, lo, hi, q, seed):
    rng = np.random.default_rng(seed)
    seq_lens = (rng.integers(lo, hi, size=n, endpoint=True) + q).astype(np.int32)
    pages = int(sum((int(L) + 15) // 16 for L in seq_lens)) + 8
    bt = D.W._assign_pages(rng, seq_lens, 16, pages)
    return D.W.Workload(name, "f16", 32, 8, 128, 16, pages, 0.3, seq_lens, np.full(n, q, np.int32), bt, seed)


CASES = {
    "f16-d128-16x[1024,8192]": lambda n: D.ragged_workload(n, "f16", 32, 8, 128, 16, 1024, 8192, 92),
    "f32-d128-16x[1024,8192]": lambda n: D.ragged_workload(n, "f32", 32, 8, 128, 16, 1024, 8192, 92),
    "f16-d128-48x[512,4096]": lambda n: D.ragged_workload(n, "f16", 32, 8, 128, 48, 512, 4096, 93),
    "f32-d64-1x512": lambda n: D.ragged_workload(n, "f32", 14, 2, 64, 1, 512, 512, 94),
    "f16-d128-24x[1024,4096]-q5": lambda n: _verify_like(n, 24, 1024, 4096, 5, 95),
}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()
    O.build()


def _forced_child(waves, dst_dir):
    """Child-process side: every case with the block shape forced (MVR_ATTN_UNIT_WAVES set by the parent)."""
    M.load_library()
    for name, mk in CASES.items():
        out, _ = D._attend(mk(name))
        np.save(os.path.join(dst_dir, f"{name}.npy"), out)
        print(f"{waves} wavefronts per block: {name} done", flush=True)


_CHILD = (
    "import sys\n"
    "sys.path[:0] = sys.argv[3].split('|')\n"
    "import test_gpu_unit_waves as T\n"
    "T._forced_child(sys.argv[1], sys.argv[2])\n"
)


@pytest.fixture(scope="module")
def forced(tmp_path_factory):
    """Outputs of every case under 1, 2 and 4 wavefronts per block, one child process per shape."""
    paths = "|".join([HERE, ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "mini-vllm-rs_amd")])
    res = {}
    for waves in ("1", "2", "4"):
        d = str(tmp_path_factory.mktemp(f"waves{waves}"))
        D.say(f"[unit-waves] child process with MVR_ATTN_UNIT_WAVES={waves}")
        child = subprocess.run([sys.executable, "-c", _CHILD, waves, d, paths],
                               env=dict(os.environ, MVR_ATTN_UNIT_WAVES=waves), capture_output=True, text=True,
                               timeout=240)
        assert child.returncode == 0, child.stdout[-2000:] + child.stderr[-2000:]
        res[waves] = {name: np.load(os.path.join(d, f"{name}.npy")) for name in CASES}
    return res


@pytest.mark.parametrize("name", list(CASES))
def test_planned_block_shape_matches_oracle(name):
    w = CASES[name](name)
    vals = D.W.host_values(w)
    got, _ = D._attend(w, vals)
    q, k, v = vals
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    D.say(f"[unit-waves] {name}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[w.dtype], err


@pytest.mark.parametrize("name", list(CASES))
def test_every_block_shape_bit_identical(name, forced):
    got, _ = D._attend(CASES[name](name))
    view = np.uint16 if got.dtype == np.float16 else np.uint32
    for waves, outs in forced.items():
        diff = int(np.count_nonzero(got.view(view) != outs[name].view(view)))
        D.say(f"[unit-waves] {name}: {diff} of {got.size} outputs differ with {waves} wavefronts per block")
        assert diff == 0, (waves, diff)
