"""Trace ranges and the checked development mode, on the GPU.

* MVR_ENABLE_ROCTX=true: every entry point runs with its roctx ranges on (the reference's span names and
  " field=value" labels, trace.rs:64-116 and nvtx_trace.rs:14-53) and its outputs are bit-identical to a run with
  them off; under rocprofv3 --marker-trace the ranges appear by name.
* MVR_ATTN_CHECKED=true: device tables that break the contract come back as the *_validate errors instead of
  being launched on; valid calls are bit-identical to unchecked ones.
* Without the checked mode, a device seq_len above max_seq_len is clamped by the kernels: the call reads only
  the block-table row's first ceil(max_seq_len / page_size) pages and equals the call at max_seq_len.

The environment flags are read once per process, hence the child processes.
"""
import glob
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mvr_attn as M  # noqa: E402
import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

EXPECTED_RANGES = [
    "attn",
    "attn-paged-fused",
    "attn-prefill-fused",
    "attn-rope tensor=query,key",
    "attn-cache operation=append",
    "attn-cache operation=access result_layout=contiguous",
    "attn-cache operation=access result_layout=repacked",
]


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()


def _child_env(**flags):
    path = os.pathsep.join([os.path.join(ROOT, "mini-vllm-rs_amd"), os.path.join(ROOT, "oracle"),
                            os.environ.get("PYTHONPATH", "")])
    env = dict(os.environ, PYTHONPATH=path)
    for k in ("MVR_ENABLE_ROCTX", "MVR_ATTN_CHECKED"):
        env.pop(k, None)
    env.update(flags)
    return env


def _run_child(mode, out_path, env, timeout=240, prefix=()):
    cmd = list(prefix) + [sys.executable, "-u", os.path.abspath(__file__), mode, out_path]
    r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=timeout)
    say(r.stdout[-3000:] + r.stderr[-3000:])
    return r


# --------------------------------------------------------------------------- child processes


def _every_entry_point(out_path):
    """Runs each entry point once on small seeded inputs and saves every output."""
    outs = {}
    # decode (split context + merge) and a prefill-sized call (prefill kernel), batched entry point
    for name, w in (("decode", W.qwen2_05b_batched_decode_f16()),
                    ("prefill", W.qwen2_7b_chunked_prefill_f16())):
        t = W.device_tensors(w, None, seed=3)
        outs[name] = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                                       t["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len)
    # page size 5: a decode call reads the pages in place; a prefill-sized call is repacked into 16-token pages
    # first
    g = torch.Generator(device="cuda").manual_seed(11)
    kp = torch.randn((40, 1, 2, 5, 64), generator=g, device="cuda").half()
    vp = torch.randn((40, 1, 2, 5, 64), generator=g, device="cuda").half()
    q = torch.randn((14, 2, 64), generator=g, device="cuda").half()
    bt = torch.arange(40, dtype=torch.int32, device="cuda").flip(0).reshape(2, 20).contiguous()
    sl = torch.tensor([97, 60], dtype=torch.int32, device="cuda")
    cu = torch.tensor([0, 1, 2], dtype=torch.int32, device="cuda")
    outs["pages5"] = M.paged_attention(q, kp, vp, bt, sl, cu, max_q_len=1, max_seq_len=97)
    q30 = torch.randn((14, 31, 64), generator=g, device="cuda").half()
    cu30 = torch.tensor([0, 30, 31], dtype=torch.int32, device="cuda")
    outs["repacked"] = M.paged_attention(q30, kp, vp, bt, sl, cu30, max_q_len=30, max_seq_len=97)
    # request-level entry
    lay = M.PagedCacheLayout(kp, vp, bt[0, :20].contiguous(), 5, 97)
    outs["request"] = M.forward_paged_attention(q[:, :1].unsqueeze(0).contiguous(), lay, 14, 2, 64, 96, 1)
    # cascade (the verify workload's prefix groups)
    w = W.llama3_8b_spec_verify_f16()
    t = W.device_tensors(w, None, seed=5)
    gcu, gpre, gbt, spre = (torch.from_numpy(x).cuda() for x in W.cascade_tables(w))
    groups = M.make_cascade_groups(gcu, gpre, gbt, spre, max_group_q_len=20, max_prefix_len=1024)
    outs["cascade"] = M.paged_attention_cascade(t["q"], t["key_pool"], t["value_pool"], t["block_tables"],
                                                t["seq_lens"], t["cu_q_lens"], groups, max_q_len=w.max_q_len,
                                                max_seq_len=w.max_seq_len)
    # gather to contiguous
    outs["gather"] = M.reconstruct_contiguous(kp, bt[1, :12].contiguous(), 60)
    # rope + append into fresh pools
    cos, sin = W.rope_tables(64, 10000.0, 128)
    kp2, vp2 = torch.zeros_like(kp), torch.zeros_like(vp)
    k_new = torch.randn((2, 2, 64), generator=g, device="cuda").half()
    v_new = torch.randn((2, 2, 64), generator=g, device="cuda").half()
    outs["rope_q"] = M.rope_append(q, k_new, v_new, torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), bt,
                                   sl, cu, kp2, vp2, max_seq_len=97)
    outs["rope_k"], outs["rope_v"] = kp2, vp2
    torch.cuda.synchronize()
    np.savez(out_path, **{k: v.cpu().numpy() for k, v in outs.items()})
    print(f"entry points done: {sorted(outs)}", flush=True)


def _checked_child(out_path):
    """MVR_ATTN_CHECKED=true: broken tables are reported, valid calls run."""
    import ctypes

    lib = M.load_library()
    results = {}
    w = W.qwen2_05b_batched_decode_f16()
    t = W.device_tensors(w, None, seed=3)
    good = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                             t["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len)
    torch.cuda.synchronize()
    results["good"] = good.cpu().numpy()

    def rc_of(**changes):
        tt = dict(t, **changes)
        try:
            M.paged_attention(tt["q"], tt["key_pool"], tt["value_pool"], tt["block_tables"], tt["seq_lens"],
                              tt["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len)
        except M.MvrError as e:
            return e.code, e.message
        return 0, ""

    long_lens = t["seq_lens"].clone()
    long_lens[3] = w.max_seq_len + 7
    results["seq_len"] = rc_of(seq_lens=long_lens)
    bad_bt = t["block_tables"].clone()
    bad_bt[2, 1] = w.num_pages + 5
    results["page_id"] = rc_of(block_tables=bad_bt)
    bad_cu = t["cu_q_lens"].clone()
    bad_cu[4] = bad_cu[3]  # an empty request
    results["empty"] = rc_of(cu_q_lens=bad_cu)
    # host hints that differ from the device tables (they would only shape the plan: checked mode reports them)
    for key, kw in (("stale_seq_lens", dict(seq_lens_host=w.seq_lens + np.int32(1), cu_q_lens_host=w.cu_q_lens)),
                    ("stale_cu_q_lens", dict(cu_q_lens_host=np.arange(w.num_seqs + 1, dtype=np.int32) * 2))):
        try:
            M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                              t["cu_q_lens"], max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, **kw)
            results[key] = (0, "")
        except M.MvrError as e:
            results[key] = (e.code, e.message)
    # a device cu_q_lens packing one token more than q holds (the last request's q_len 2): q is a view one token
    # short of the tensor it views and out is full-size, so every address the kernel could touch lies in
    # allocated memory, should the check miss
    q_big = torch.zeros((t["q"].shape[0], w.total_q + 1, t["q"].shape[2]), dtype=t["q"].dtype, device="cuda")
    out_big = torch.empty_like(q_big)
    cu_more = t["cu_q_lens"].clone()
    cu_more[-1] += 1
    try:
        M.paged_attention(q_big[:, :w.total_q], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"],
                          cu_more, out_big, max_q_len=2, max_seq_len=w.max_seq_len)
        results["short_q"] = (0, "")
    except M.MvrError as e:
        results["short_q"] = (e.code, e.message)
    # rope + append writing a page outside the pool
    cos, sin = W.rope_tables(64, 10000.0, w.max_seq_len)
    q = t["q"]
    k_new = torch.zeros((2, w.total_q, 64), dtype=torch.float16, device="cuda")
    bt_rope = t["block_tables"].clone()
    last = (int(w.seq_lens[0]) - 1) // 16
    bt_rope[0, last] = -1
    try:
        M.rope_append(q, k_new, k_new, torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), bt_rope,
                      t["seq_lens"], t["cu_q_lens"], t["key_pool"], t["value_pool"], max_seq_len=w.max_seq_len)
        results["rope_page"] = (0, "")
    except M.MvrError as e:
        results["rope_page"] = (e.code, e.message)
    # cascade: a member whose first page differs from its group's
    v = W.llama3_8b_spec_verify_f16()
    tv = W.device_tensors(v, None, seed=5)
    gcu, gpre, gbt, spre = W.cascade_tables(v)
    gbt = gbt.copy()
    gbt[1, 3] = (gbt[1, 3] + 1) % v.num_pages
    groups = M.make_cascade_groups(*(torch.from_numpy(x).cuda() for x in (gcu, gpre, gbt, spre)),
                                   max_group_q_len=20, max_prefix_len=1024)
    try:
        M.paged_attention_cascade(tv["q"], tv["key_pool"], tv["value_pool"], tv["block_tables"], tv["seq_lens"],
                                  tv["cu_q_lens"], groups, max_q_len=v.max_q_len, max_seq_len=v.max_seq_len)
        results["cascade_page"] = (0, "")
    except M.MvrError as e:
        results["cascade_page"] = (e.code, e.message)
    torch.cuda.synchronize()
    codes = {k: v for k, v in results.items() if k != "good"}
    print(f"checked results: {codes}", flush=True)
    np.savez(out_path, good=results["good"],
             **{k: np.array([v[0]]) for k, v in codes.items()},
             **{k + "_msg": np.array([v[1]]) for k, v in codes.items()})
    del lib, ctypes


# --------------------------------------------------------------------------- tests


def test_roctx_ranges_leave_every_entry_point_bit_identical():
    with tempfile.TemporaryDirectory() as d:
        off, on = os.path.join(d, "off.npz"), os.path.join(d, "on.npz")
        assert _run_child("entry-points", off, _child_env(MVR_ENABLE_ROCTX="false")).returncode == 0
        assert _run_child("entry-points", on, _child_env(MVR_ENABLE_ROCTX="true")).returncode == 0
        a, b = np.load(off), np.load(on)
        assert sorted(a.files) == sorted(b.files) and len(a.files) == 10
        for k in a.files:
            assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), k


def test_roctx_ranges_appear_in_a_marker_trace():
    prof = shutil.which("rocprofv3")
    if prof is None:
        pytest.skip("rocprofv3 is not installed")
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "on.npz")
        tdir = os.path.join(d, "trace")
        r = _run_child("entry-points", out, _child_env(MVR_ENABLE_ROCTX="true", TMPDIR=d), timeout=400,
                       prefix=(prof, "--marker-trace", "--output-format", "csv", "-d", tdir, "-o", "mvr", "--"))
        # The profiler itself may end with a non-zero status after the program finished; the program's own end
        # is its output file and its last line.
        assert os.path.exists(out) and "entry points done" in r.stdout, r.returncode
        files = glob.glob(os.path.join(tdir, "**", "*marker_api_trace.csv"), recursive=True)
        assert files, os.listdir(tdir) if os.path.isdir(tdir) else "no trace directory"
        text = "".join(open(f).read() for f in files)
        missing = [n for n in EXPECTED_RANGES if f'"{n}"' not in text and f",{n}," not in text]
        assert not missing, missing


def test_checked_mode_reports_broken_tables_and_runs_valid_calls():
    with tempfile.TemporaryDirectory() as d:
        ref, chk = os.path.join(d, "ref.npz"), os.path.join(d, "chk.npz")
        assert _run_child("entry-points", ref, _child_env()).returncode == 0
        assert _run_child("checked", chk, _child_env(MVR_ATTN_CHECKED="true")).returncode == 0
        a, c = np.load(ref), np.load(chk)
        assert np.array_equal(a["decode"].view(np.uint16), c["good"].view(np.uint16))
        assert int(c["seq_len"][0]) == M.MVR_E_INVALID_ARGUMENT and "max_seq_len" in str(c["seq_len_msg"][0])
        assert int(c["page_id"][0]) == M.MVR_E_PAGE_ID and "outside a pool" in str(c["page_id_msg"][0])
        assert int(c["empty"][0]) == M.MVR_E_INVALID_ARGUMENT and "at least one token" in str(c["empty_msg"][0])
        assert int(c["stale_seq_lens"][0]) == M.MVR_E_INVALID_ARGUMENT and "seq_lens_host" in str(
            c["stale_seq_lens_msg"][0])
        assert int(c["stale_cu_q_lens"][0]) == M.MVR_E_INVALID_ARGUMENT and "cu_q_lens_host" in str(
            c["stale_cu_q_lens_msg"][0])
        assert int(c["short_q"][0]) == M.MVR_E_INVALID_ARGUMENT and "exceeds total_q" in str(c["short_q_msg"][0])
        assert int(c["rope_page"][0]) == M.MVR_E_PAGE_ID
        assert int(c["cascade_page"][0]) == M.MVR_E_INVALID_ARGUMENT and "differs" in str(c["cascade_page_msg"][0])


@pytest.mark.parametrize("make", [W.qwen2_05b_batched_decode_f16, W.qwen2_7b_chunked_prefill_f16],
                         ids=["decode", "prefill"])
def test_seq_len_above_max_seq_len_is_clamped(make):
    """A device seq_len above max_seq_len (a broken contract, no checked mode) reads no page past the
    first ceil(max_seq_len / page_size) entries of its row: entries after them hold ids outside the pool, and
    the call equals the one whose seq_len is max_seq_len, bit for bit."""
    w = make()
    t = W.device_tensors(w, None, seed=9)
    b = int(np.argmax(w.seq_lens))
    pages = -(-w.max_seq_len // w.page_size)
    extra = 4
    bt = torch.full((w.num_seqs, w.block_tables.shape[1] + extra), 2 ** 30, dtype=torch.int32, device="cuda")
    bt[:, :w.block_tables.shape[1]] = t["block_tables"]
    bt[b, pages:] = 2 ** 30  # never read: past max_seq_len
    long_lens = t["seq_lens"].clone()
    long_lens[b] = w.max_seq_len + extra * w.page_size
    q_len = int(w.q_lens[b])
    cu = t["cu_q_lens"]
    ref = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], bt, t["seq_lens"], cu, max_q_len=w.max_q_len,
                            max_seq_len=w.max_seq_len)
    got = M.paged_attention(t["q"], t["key_pool"], t["value_pool"], bt, long_lens, cu, max_q_len=w.max_q_len,
                            max_seq_len=w.max_seq_len)
    torch.cuda.synchronize()
    assert q_len >= 1
    assert torch.equal(ref, got)


if __name__ == "__main__" and len(sys.argv) > 2:
    mode, path = sys.argv[1], sys.argv[2]
    if mode == "entry-points":
        _every_entry_point(path)
    elif mode == "checked":
        _checked_child(path)
