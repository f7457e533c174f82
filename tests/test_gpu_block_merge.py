"""GPU parity of the block-merge launch of the split-context kernel.

When a uniform batch splits every context into at most one block's worth of
partitions (blocks of 4, 8 or 16 wavefronts, at least three quarters of them
holding a partition), the planner puts the partitions of one (sequence, KV
head) in one block and merges them through LDS instead of writing fp32
partials and launching the merge kernel.  The plan is visible from the host:
such a call needs no workspace.  Same bar as every call: 2e-3 (F16) / 1e-5 (F32)
against the oracle.  Covers F16 at head_dim 128 (the batch-64 decode shape at
1K tokens), ragged lengths planned as uniform (no length hint), so that short
sequences leave partitions without keys that still join the block's merge,
and F32 at head_dim 64.  The block-merge launch is also compared bit for bit
with the two-launch plan (fp32 partials in the workspace, merge kernel) on the
same batch, computed in a child process with MVR_ATTN_BLOCK_MERGE=false (the
flag is read once per process): both merge the same partition states with the
same weights in the same order.  The wider blocks are pinned the same way on
a 512-token F16 sequence (16 partitions, the planner's own choice) and, with
MVR_ATTN_CHUNKS_PER_PARTITION fixing the split in both child processes, on
8 partitions at head_dim 128, 16 at head_dim 64 and 3 partitions in a
4-wavefront block (one wavefront without keys), F16 and F32 (F32 takes no
wider block than 4).
"""
import math
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


def decode_workload(name, dtype, hq, hkv, d, lens, seed, page_size=16):
    rng = np.random.default_rng(seed)
    seq_lens = np.asarray(lens, np.int32)
    need = [math.ceil(int(L) / page_size) for L in seq_lens]
    num_pages = sum(need) + 4
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((len(need), max(need)), np.int32)
    used = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[used:used + n]
        used += n
    return W.Workload(name, dtype, hq, hkv, d, page_size, num_pages, 0.3, seq_lens, np.ones(len(need), np.int32), bt,
                      seed)


def run_and_check(w, hint):
    vals = W.host_values(w)
    t = W.device_tensors(w, vals)
    sum_hint = int(w.seq_lens.sum()) if hint else 0
    args = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                       t["q"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=sum_hint)
    assert M.workspace_size(args) == 0, "expected the block-merge plan (no workspace)"
    out = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                            max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=sum_hint)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    q, k, v = vals
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got - ref).max())
    say(f"[block-merge] {w.name}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[w.dtype], err


def test_uniform_f16_d128():
    run_and_check(decode_workload("f16 D128 64 x 1024", "f16", 32, 8, 128, [1024] * 64, 61), hint=True)


def test_ragged_lengths_planned_uniform():
    rng = np.random.default_rng(62)
    lens = rng.integers(16, 1024, size=64, endpoint=True)
    lens[0] = 1024  # max_seq_len 1024: 4 partitions of 256 tokens, most sequences leave some without keys
    run_and_check(decode_workload("f16 D128 64 x U[16,1024] without hint", "f16", 32, 8, 128, lens, 62), hint=False)


def test_uniform_f32_d64():
    run_and_check(decode_workload("f32 D64 256 x 512", "f32", 14, 2, 64, [512] * 256, 63), hint=True)


def _uniform_f16_workload():
    return decode_workload("f16 D128 64 x 1024", "f16", 32, 8, 128, [1024] * 64, 61)


def _attend(w):
    t = W.device_tensors(w, W.host_values(w))
    args = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                       t["q"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    need = M.workspace_size(args)
    out = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                            max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    torch.cuda.synchronize()
    return out.cpu().numpy(), need


def _two_launch_child(path):
    """Child-process side: the same batch with block merge switched off."""
    M.load_library()
    out, need = _attend(_uniform_f16_workload())
    assert need > 0, "expected the two-launch plan (fp32 partials in the workspace)"
    np.save(path, out)


_CHILD = (
    "import sys\n"
    "sys.path[:0] = sys.argv[2].split('|')\n"
    "import test_gpu_block_merge as T\n"
    "T._two_launch_child(sys.argv[1])\n"
    "print('two-launch plan done', flush=True)\n"
)


def test_bit_identical_to_two_launch_plan(tmp_path):
    w = _uniform_f16_workload()
    got, need = _attend(w)
    assert need == 0, "expected the block-merge plan (no workspace)"
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = "|".join([here, root, os.path.join(root, "oracle"), os.path.join(root, "mini-vllm-rs_amd")])
    dst = str(tmp_path / "two_launch.npy")
    say("[block-merge] two-launch plan in a child process (MVR_ATTN_BLOCK_MERGE=false)")
    child = subprocess.run([sys.executable, "-c", _CHILD, dst, paths], env=dict(os.environ, MVR_ATTN_BLOCK_MERGE="false"),
                           capture_output=True, text=True, timeout=180)
    assert child.returncode == 0, child.stdout[-2000:] + child.stderr[-2000:]
    two = np.load(dst)
    assert got.dtype == np.float16 and two.dtype == np.float16 and got.shape == two.shape
    diff = int(np.count_nonzero(got.view(np.uint16) != two.view(np.uint16)))
    say(f"[block-merge] {w.name}: {diff} of {got.size} outputs differ from the two-launch plan")
    assert diff == 0


# Wider blocks: (name, builder, chunks per partition or None for the planner's choice).
WIDE = {
    "f16 D64 1 x 512 (16 partitions)": (lambda: decode_workload("f16 D64 1 x 512", "f16", 14, 2, 64, [512], 64), None),
    "f32 D64 1 x 400 (3 of 4 partitions)": (lambda: decode_workload("f32 D64 1 x 400", "f32", 14, 2, 64, [400], 68),
                                            9),
    "f16 D128 4 x 1024 (8 partitions)": (lambda: decode_workload("f16 D128 4 x 1024", "f16", 32, 8, 128, [1024] * 4, 65),
                                         8),
    "f16 D64 2 x 1000 (16 partitions)": (lambda: decode_workload("f16 D64 2 x 1000", "f16", 14, 2, 64, [1000] * 2, 66),
                                         4),
    "f16 D128 1 x 768 (3 of 4 partitions)": (lambda: decode_workload("f16 D128 1 x 768", "f16", 32, 8, 128, [768], 67),
                                             16),
}


def _wide_child(path, key):
    """Child-process side: the workload under this process's environment; saves the output and the workspace need."""
    M.load_library()
    out, need = _attend(WIDE[key][0]())
    np.save(path, out)
    np.save(path + ".need.npy", np.array([need], np.int64))


_WIDE_CHILD = (
    "import sys\n"
    "sys.path[:0] = sys.argv[3].split('|')\n"
    "import test_gpu_block_merge as T\n"
    "T._wide_child(sys.argv[1], sys.argv[2])\n"
    "print('done', flush=True)\n"
)


def _run_child(tmp_path, key, tag, env):
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = "|".join([here, root, os.path.join(root, "oracle"), os.path.join(root, "mini-vllm-rs_amd")])
    dst = str(tmp_path / f"{tag}.npy")
    child = subprocess.run([sys.executable, "-c", _WIDE_CHILD, dst, key, paths], env=dict(os.environ, **env),
                           capture_output=True, text=True, timeout=180)
    assert child.returncode == 0, child.stdout[-2000:] + child.stderr[-2000:]
    return np.load(dst), int(np.load(dst + ".need.npy")[0])


@pytest.mark.parametrize("key", sorted(WIDE))
def test_wide_blocks_match_oracle_and_two_launch_plan(tmp_path, key):
    build, cpp = WIDE[key]
    w = build()
    env = {} if cpp is None else {"MVR_ATTN_CHUNKS_PER_PARTITION": str(cpp)}
    say(f"[block-merge] {key}: block-merge and two-launch plans in child processes")
    got, need = _run_child(tmp_path, key, "bm", dict(env, MVR_ATTN_BLOCK_MERGE="true"))
    two, need2 = _run_child(tmp_path, key, "two", dict(env, MVR_ATTN_BLOCK_MERGE="false"))
    assert need == 0, "expected the block-merge plan (no workspace)"
    assert need2 > 0, "expected the two-launch plan (fp32 partials in the workspace)"
    vals = W.host_values(w)
    q, k, v = vals
    ref = O.paged_attention(q, k, v, w.block_tables, w.seq_lens, w.cu_q_lens, w.num_q_heads, w.num_kv_heads,
                            w.head_dim, w.page_size, dtype=O.F16 if w.dtype == "f16" else O.F32, num_threads=16)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    say(f"[block-merge] {key}: max-abs vs oracle {err:.3e}")
    assert np.isfinite(got).all() and err <= TOL[w.dtype], err
    view = np.uint16 if w.dtype == "f16" else np.uint32
    diff = int(np.count_nonzero(got.view(view) != two.view(view)))
    say(f"[block-merge] {key}: {diff} of {got.size} outputs differ from the two-launch plan")
    assert diff == 0
