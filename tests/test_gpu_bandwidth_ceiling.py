"""HBM read ceilings of the part and the headline decode call against them.

The headline's roofline fraction is quoted against the published 8 TB/s;
this test measures what the part actually delivers to the two access
patterns that matter here (tests/bandwidth/hbm_read_probe.hip): one linear
pass over 2 GiB, and the same bytes as 4 KiB pages (one KV head's slab of a
16-token F16 page at head_dim 128) visited in a random order, one wavefront
per page, as a paged K/V walk reads them.  Each probe is swept over grid
sizes and bytes in flight (4, 8, 16 loads per thread for the linear pass;
2, 4, 8 pages per wavefront for the walk), 10 timed launches each (HIP
events), so that the best rate is a plateau and not a probe that stops
short of the ceiling.  The Llama-3-8B batch-64 x 8K F16 decode call (its
algorithmic K/V + Q + output bytes) must then reach at least 80% of the
page-walk ceiling: a loose bar, so that the box-to-box spread of either
figure cannot fail it, while a plan or kernel regression of the headline
would.
"""
import ctypes
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mvr_attn as M  # noqa: E402
import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE = os.path.join(HERE, "bandwidth", "libhbm_read_probe.so")
BYTES = 2 << 30
PAGE = 4096
GRIDS = (1024, 2048, 4096, 8192, 16384)
STREAM_INFLIGHT = (4, 8, 16)
WALK_INFLIGHT = (2, 4, 8)


@pytest.fixture(scope="module")
def probe():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not os.path.exists(PROBE):
        pytest.fail(f"{PROBE} is missing: build it with `make -C {os.path.dirname(PROBE)}`")
    lib = ctypes.CDLL(PROBE)
    lib.hbm_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
    lib.hbm_page_walk_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_void_p]
    return lib


def _rate(launch, nbytes):
    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        launch()
    e1.record()
    e1.synchronize()
    return nbytes * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9  # GB/s


def test_headline_reaches_the_page_walk_ceiling(probe):
    buf = torch.zeros(BYTES, dtype=torch.uint8, device="cuda")
    n_pages = BYTES // PAGE
    order_h = np.random.default_rng(7).permutation(n_pages).astype(np.int32)
    assert order_h.min() == 0 and order_h.max() == n_pages - 1  # every id in bounds
    order = torch.from_numpy(order_h).cuda()
    out = torch.empty(max(GRIDS) * 256, dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    stream_gbs, walk_gbs = {}, {}
    for grid in GRIDS:
        assert out.numel() >= grid * 256
        for k in STREAM_INFLIGHT:
            rc = []
            stream_gbs[grid, k] = _rate(lambda: rc.append(probe.hbm_stream_read(buf.data_ptr(), BYTES, out.data_ptr(),
                                                                                grid, k, stream)), BYTES)
            assert set(rc) == {0}, rc
        for k in WALK_INFLIGHT:
            rc = []
            walk_gbs[grid, k] = _rate(lambda: rc.append(probe.hbm_page_walk_read(buf.data_ptr(), order.data_ptr(),
                                                                                 n_pages, out.data_ptr(), grid, k,
                                                                                 stream)), BYTES)
            assert set(rc) == {0}, rc
        print(f"[ceiling] grid {grid:5d}: linear " +
              ", ".join(f"{k:2d}/thread {stream_gbs[grid, k]:6.0f}" for k in STREAM_INFLIGHT) +
              " GB/s; page walk " + ", ".join(f"{k}/wave {walk_gbs[grid, k]:6.0f}" for k in WALK_INFLIGHT) + " GB/s",
              flush=True)
    del buf, order, out
    torch.cuda.empty_cache()
    best_stream, best_walk = max(stream_gbs.values()), max(walk_gbs.values())

    w = W.llama3_8b_decode_b64_8k_f16()
    t = W.device_tensors(w, None, seed=3)
    o = torch.empty_like(t["q"])
    a = M.make_args(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"], o,
                    max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()))
    assert M.workspace_size(a) == 0  # the block-merge launch
    lib = M.load_library()
    headline = _rate(lambda: lib.mvr_paged_attention(ctypes.byref(a)), w.algorithmic_bytes())
    print(f"[ceiling] best linear {best_stream:.0f} GB/s, best page walk {best_walk:.0f} GB/s; headline decode "
          f"{headline:.0f} GB/s = {headline / best_walk:.1%} of the page walk, {headline / 8000:.1%} of 8 TB/s",
          flush=True)
    assert best_walk > 3000 and best_stream > 3000, (best_walk, best_stream)
    assert headline >= 0.8 * best_walk, (headline, best_walk)
