"""Concurrent callers on one GPU.

The reference runs one backend per OS thread (server/mod.rs:380-391), and
the library keeps no mutable global state, so calls from several host
threads on their own streams, each with its own workspace, must give exactly
the results of the same calls made one after another.  Four workloads that
take different kernels (split decode with its merge for config 1, ragged
F16 D=64 decode for config 2, the chunked-prefill kernel for config 4, and
32-row verify tiles for config 5) run in four threads, 20 calls each, on
four default-priority streams, and every output is compared bit for bit
with a sequential run of the same call.
"""
import os
import sys
import threading

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (ROOT, os.path.join(ROOT, "mini-vllm-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

torch = pytest.importorskip("torch")
import mvr_attn as M  # noqa: E402
import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    M.load_library()


def _call(w, t, stream=None):
    return M.paged_attention(t["q"], t["key_pool"], t["value_pool"], t["block_tables"], t["seq_lens"], t["cu_q_lens"],
                             max_q_len=w.max_q_len, max_seq_len=w.max_seq_len, stream=stream,
                             sum_seq_lens=int(w.seq_lens.sum()))


def test_threads_on_separate_streams_match_sequential_calls():
    cfgs = [1, 2, 4, 5]
    work = []
    for c in cfgs:
        w = W.CONFIGS[c]()
        work.append((c, w, W.device_tensors(w, None)))
    expected = {c: _call(w, t).cpu().numpy() for c, w, t in work}
    torch.cuda.synchronize()
    print(f"[concurrency] sequential outputs for configs {cfgs}", flush=True)

    results, errors = {}, []
    start = threading.Barrier(len(work))

    def worker(c, w, t):
        try:
            stream = torch.cuda.Stream()
            outs = []
            start.wait()
            with torch.cuda.stream(stream):
                for _ in range(20):
                    outs.append(_call(w, t, stream=stream))
            stream.synchronize()
            results[c] = [o.cpu().numpy() for o in outs]
        except Exception as e:  # reported by the main thread
            errors.append((c, repr(e)))

    threads = [threading.Thread(target=worker, args=item) for item in work]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for c, _, _ in work:
        ref = expected[c]
        view = np.uint16 if ref.dtype == np.float16 else np.uint32
        bad = sum(int(np.count_nonzero(o.view(view) != ref.view(view))) for o in results[c])
        print(f"[concurrency] config {c}: {len(results[c])} concurrent calls, {bad} outputs differ", flush=True)
        assert bad == 0
