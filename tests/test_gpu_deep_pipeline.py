"""GPU parity of the deep pipeline (three K/V chunks in flight per wavefront).

Ragged batches of few sequences keep the slot == partition layout, and their
live wavefronts do not fill the device, so the planner gives them the kernel
instantiation with three chunks in flight instead of two (deep_pipeline: one
16-row tile, D * element size <= 256 bytes, at least 8 chunks per partition).
These cases take it by that rule:
  * 16 F16 sequences of 1,900..14,800 tokens, 32/8 heads, D=128 (about 38
    chunks per partition);
  * 8 F16 sequences of 8K..32K tokens, 14/2 heads, D=64 (about 13);
  * 6 F32 sequences of 16K..40K tokens, 14/2 heads, D=64 (about 13).
Same bar as every call: 2e-3 (F16) / 1e-5 (F32) against the oracle.  The
pipeline depth changes only when loads are issued, not the arithmetic, so
the result is also compared bit for bit with the two-chunk pipeline of the
same batch, computed in a child process with MVR_ATTN_DEEP_PIPELINE=false
(the flag is read once per process).
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

CASES = {
    "f16-d128-16x[1900,14800]": ("f16", 32, 8, 128, 16, 1900, 14800, 81),
    "f16-d64-8x[8000,32000]": ("f16", 14, 2, 64, 8, 8000, 32000, 82),
    "f32-d64-6x[16000,40000]": ("f32", 14, 2, 64, 6, 16000, 40000, 83),
}


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()
    O.build()


def _case(name):
    return D.ragged_workload(name, *CASES[name])


@pytest.mark.parametrize("name", list(CASES))
def test_deep_pipeline_matches_oracle(name):
    w = _case(name)
    vals = D.W.host_values(w)
    got, _ = D._attend(w, vals)
    q, k, v = vals
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    D.say(f"[deep] {name}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[w.dtype], err


def _two_chunk_child(name, path):
    """Child-process side: the same batch with the deep pipeline switched off."""
    M.load_library()
    out, _ = D._attend(_case(name))
    np.save(path, out)


_CHILD = (
    "import sys\n"
    "sys.path[:0] = sys.argv[3].split('|')\n"
    "import test_gpu_deep_pipeline as T\n"
    "T._two_chunk_child(sys.argv[1], sys.argv[2])\n"
    "print('two-chunk pipeline done', flush=True)\n"
)


@pytest.mark.parametrize("name", list(CASES))
def test_deep_pipeline_bit_identical_to_two_chunks(name, tmp_path):
    got, _ = D._attend(_case(name))
    paths = "|".join([HERE, ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "mini-vllm-rs_amd")])
    dst = str(tmp_path / "two_chunks.npy")
    D.say(f"[deep] {name}: two chunks in flight in a child process (MVR_ATTN_DEEP_PIPELINE=false)")
    child = subprocess.run([sys.executable, "-c", _CHILD, name, dst, paths],
                           env=dict(os.environ, MVR_ATTN_DEEP_PIPELINE="false"), capture_output=True, text=True,
                           timeout=180)
    assert child.returncode == 0, child.stdout[-2000:] + child.stderr[-2000:]
    ref = np.load(dst)
    view = np.uint16 if got.dtype == np.float16 else np.uint32
    diff = int(np.count_nonzero(got.view(view) != ref.view(view)))
    D.say(f"[deep] {name}: {diff} of {got.size} outputs differ from the two-chunk pipeline")
    assert diff == 0
