"""Benchmark: page-wise decode attention on one MI355X.

Headline workload: Llama-3-8B-shape decode, batch 64 x 8192-token contexts,
32 Q / 8 KV heads, head_dim 128, F16, 16-token pages randomly permuted in a
32768-page pool.  One step = one batched attention call over the whole batch
(one layer, one decode step), inputs resident in HBM.  Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--skip-cpu] [--only-headline]
"""
import argparse
import ctypes
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mini-vllm-rs_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
MFMA_F32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA
# HBM bytes per launch of the headline's kernel, from the FETCH_SIZE / WRITE_SIZE counter runs summarised in
# this file (line "bytes_per_launch: N"), valid for the kernel sources it names (line "source_sha256: H", the
# SHA-256 of TRAFFIC_SOURCES concatenated): after any change to them the figure is stale and not reported.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "paged_attention_decode_b64_ctx8192_f16_hbm_traffic.md")
TRAFFIC_SOURCES = [os.path.join(ROOT, "mini-vllm-rs_amd", "csrc", f)
                   for f in ("paged_attention.hip", "paged_attention_kernels.hpp")]


def traffic_source_sha256():
    import hashlib

    h = hashlib.sha256()
    for f in TRAFFIC_SOURCES:
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Runner:
    """Prebuilt C argument block for repeated calls (no per-call Python work beyond one ctypes call).
    host_hints: also pass host copies of seq_lens / cu_q_lens (the planner's optional hints)."""

    def __init__(self, w, tensors, torch, M, host_hints=False):
        self.w = w
        self.t = tensors
        self.out = torch.empty_like(tensors["q"])
        hints = dict(seq_lens_host=w.seq_lens, cu_q_lens_host=w.cu_q_lens) if host_hints else {}
        self.args = M.make_args(tensors["q"], tensors["key_pool"], tensors["value_pool"], tensors["block_tables"],
                                tensors["seq_lens"], tensors["cu_q_lens"], self.out, max_q_len=w.max_q_len,
                                max_seq_len=w.max_seq_len, sum_seq_lens=int(w.seq_lens.sum()), **hints)
        need = M.workspace_size(self.args)
        self.ws = M.new_workspace(need, "cuda")
        self.args.workspace = self.ws.data_ptr()
        self.args.workspace_bytes = need
        self.lib = M.load_library()
        self.M = M

    def step(self):
        rc = self.lib.mvr_paged_attention(ctypes.byref(self.args))
        if rc != 0:
            raise self.M.MvrError(rc, self.lib.mvr_last_error().decode())


def time_steps(runner, torch, steps, warmup):
    for _ in range(warmup):
        runner.step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        runner.step()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))  # microseconds, kernel-side
    return wall, per


def cpu_model():
    """The host CPU's model name (first "model name" line of /proc/cpuinfo) and its logical CPU count."""
    name = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(model=name, logical_cpus=os.cpu_count(), usable_cpus=len(os.sched_getaffinity(0)))


def cpu_baseline(W):
    """The oracle (C restatement of forward_paged_attention, reference dataflow with f16-rounded
    intermediates) on the headline workload itself (64 sequences x 8 kv heads x 8192 tokens), repeated for
    about 10 s on the host cores available to this process (at most 16).  Reported in the headline unit
    (effective KV-read GB/s)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import oracle

    oracle.build()
    full = W.llama3_8b_decode_b64_8k_f16()
    sample = full
    q, k, v = W.host_values(sample)
    threads = min(len(os.sched_getaffinity(0)), 16)
    reps = 0
    t0 = time.perf_counter()
    while True:
        oracle.paged_attention(q, k, v, sample.block_tables, sample.seq_lens, sample.cu_q_lens, sample.num_q_heads,
                               sample.num_kv_heads, sample.head_dim, sample.page_size, dtype=oracle.F16,
                               num_threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el > 10.0:
            break
    per_call = el / reps
    gbs = sample.algorithmic_bytes() / per_call / 1e9
    # The same dataflow on one thread, on one sequence (all 8 kv heads, 8192 tokens), for about 5 s.
    one = W.llama3_8b_decode_b64_8k_f16(batch=1)
    q1, k1, v1 = W.host_values(one)
    reps1 = 0
    t0 = time.perf_counter()
    while True:
        oracle.paged_attention(q1, k1, v1, one.block_tables, one.seq_lens, one.cu_q_lens, one.num_q_heads,
                               one.num_kv_heads, one.head_dim, one.page_size, dtype=oracle.F16, num_threads=1)
        reps1 += 1
        el1 = time.perf_counter() - t0
        if el1 > 5.0:
            break
    per_call1 = el1 / reps1
    del q, k, v, q1, k1, v1
    return dict(value=round(gbs, 3), unit="GB/s", cores=threads, kind="port",
                sample=f"the whole batch: {full.num_seqs} sequences x 8 kv heads x 8192 tokens (F16 reference "
                       f"dataflow), {reps} calls, {per_call * 1e3:.1f} ms/call",
                single_thread=dict(value=round(one.algorithmic_bytes() / per_call1 / 1e9, 3), unit="GB/s", cores=1,
                                   sample=f"1 of {full.num_seqs} sequences x 8 kv heads x 8192 tokens, {reps1} calls, "
                                          f"{per_call1 * 1e3:.1f} ms/call"),
                host=cpu_model())


def measure(W, M, torch, cfg, steps, warmup):
    """cfg: a key of W.CONFIGS or a workload builder.  The call carries the host copies of the length tables,
    as the reference's runner has them (prepare_forward builds them on the host before uploading); a
    prefill-sized batch of several sequences is also timed without them (no_hints_us_median)."""
    w = W.CONFIGS[cfg]() if isinstance(cfg, int) else cfg()
    t = W.device_tensors(w, None)
    prefill_sized = w.total_q > w.num_seqs * 16
    no_hints = None
    if prefill_sized and w.num_seqs > 1:
        _, per_nh = time_steps(Runner(w, t, torch, M), torch, steps, warmup)
        no_hints = round(per_nh[len(per_nh) // 2], 2)
    r = Runner(w, t, torch, M, host_hints=True)
    wall, per = time_steps(r, torch, steps, warmup)
    med = per[len(per) // 2]
    mean = sum(per) / len(per)
    res = dict(workload=w.name, us_per_step_median=round(med, 2), us_per_step_mean=round(mean, 2),
               wall_us_per_step=round(wall / steps * 1e6, 2), bytes=w.algorithmic_bytes(),
               eff_gbs=round(w.algorithmic_bytes() / (med * 1e-6) / 1e9, 1))
    if w.shared_pages:
        res["unique_bytes"] = w.algorithmic_bytes(unique=True)
        res["unique_gbs"] = round(w.algorithmic_bytes(unique=True) / (med * 1e-6) / 1e9, 1)
        res["hbm_frac"] = round(res["unique_gbs"] / HBM_PEAK_GBS, 4)
    else:
        res["hbm_frac"] = round(res["eff_gbs"] / HBM_PEAK_GBS, 4)
    if no_hints is not None:
        res["no_hints_us_median"] = no_hints
    if prefill_sized:  # MFMA-bound
        peak = MFMA_F16_PEAK_TFLOPS if w.dtype == "f16" else MFMA_F32_PEAK_TFLOPS
        res["tflops"] = round(w.flops() / (med * 1e-6) / 1e12, 2)
        res["mfma_frac"] = round(res["tflops"] / peak, 4)
        res["mfma_peak_tflops"] = peak
    del t, r
    torch.cuda.empty_cache()
    return res


class AppendRunner:
    """RoPE + KV-page append for the new tokens of a workload (its block tables and pools), prebuilt args."""

    def __init__(self, w, tensors, torch, M, W):
        import numpy as np

        g = torch.Generator(device="cuda").manual_seed(w.seed)
        T, d = w.total_q, w.head_dim
        dt = torch.float16 if w.dtype == "f16" else torch.float32
        self.q = (torch.randn((w.num_q_heads, T, d), generator=g, device="cuda") * 0.3).to(dt)
        self.k = (torch.randn((w.num_kv_heads, T, d), generator=g, device="cuda") * 0.3).to(dt)
        self.v = (torch.randn((w.num_kv_heads, T, d), generator=g, device="cuda") * 0.3).to(dt)
        cos, sin = W.rope_tables(d, 10000.0, w.max_seq_len, np.float16 if w.dtype == "f16" else np.float32)
        self.cos, self.sin = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        self.q_out = torch.empty_like(self.q)
        self.args = M.make_rope_append_args(self.q, self.k, self.v, self.cos, self.sin, tensors["block_tables"],
                                            tensors["seq_lens"], tensors["cu_q_lens"], tensors["key_pool"],
                                            tensors["value_pool"], self.q_out, max_seq_len=w.max_seq_len)
        self.lib = M.load_library()
        self.M = M
        es = 2 if w.dtype == "f16" else 4
        # Q read + written, K read + written, V read + written, one cos and one sin row, one page id per token.
        self.bytes = T * ((w.num_q_heads + 2 * w.num_kv_heads) * d * es * 2 + d * es + 4)

    def step(self):
        rc = self.lib.mvr_rope_append(ctypes.byref(self.args))
        if rc != 0:
            raise self.M.MvrError(rc, self.lib.mvr_last_error().decode())


class CascadeRunner(Runner):
    """The workload's call through mvr_paged_attention_cascade with its prefix groups."""

    def __init__(self, w, tensors, torch, M, W):
        super().__init__(w, tensors, torch, M)
        gcu, gpre, gbt, spre = W.cascade_tables(w)
        self.dev = [torch.from_numpy(x).cuda() for x in (gcu, gpre, gbt, spre)]
        self.groups = M.make_cascade_groups(*self.dev, max_group_q_len=int(max(gcu[1:] - gcu[:-1])),
                                            max_prefix_len=int(gpre.max()), sum_prefix_lens=int(spre.sum()))
        need = self.lib.mvr_paged_attention_cascade_workspace_size(ctypes.byref(self.args), ctypes.byref(self.groups))
        self.ws = M.new_workspace(need, "cuda")
        self.args.workspace = self.ws.data_ptr()
        self.args.workspace_bytes = need

    def step(self):
        rc = self.lib.mvr_paged_attention_cascade(ctypes.byref(self.args), ctypes.byref(self.groups))
        if rc != 0:
            raise self.M.MvrError(rc, self.lib.mvr_last_error().decode())


def measure_cascade(W, M, torch, cfg, steps, warmup, with_plain=False):
    """cfg: a key of W.CONFIGS or a workload builder.  with_plain: also time the plain call on the same
    tensors, for the speedup."""
    w = W.CONFIGS[cfg]() if isinstance(cfg, int) else cfg()
    t = W.device_tensors(w, None)
    r = CascadeRunner(w, t, torch, M, W)
    wall, per = time_steps(r, torch, steps, warmup)
    med = per[len(per) // 2]
    ub = w.algorithmic_bytes(unique=True)
    res = dict(workload=f"{w.name} through cascade attention ({len(w.prefix_groups)} prefix groups)",
               us_per_step_median=round(med, 2), unique_bytes=ub, unique_gbs=round(ub / (med * 1e-6) / 1e9, 1),
               hbm_frac=round(ub / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
    if with_plain:
        del r
        p = Runner(w, t, torch, M)
        _, per_p = time_steps(p, torch, steps, warmup)
        med_p = per_p[len(per_p) // 2]
        res.update(plain_us_per_step_median=round(med_p, 2), speedup_vs_plain=round(med_p / med, 3),
                   logical_bytes=w.algorithmic_bytes())
        r = p
    del t, r
    torch.cuda.empty_cache()
    return res


class SliceRunner(Runner):
    """The call over sequences [lo, hi) of a workload alone, on the same device tensors (q / out rows of those
    sequences; block-table rows; lengths; cu_q_lens rebased to 0)."""

    def __init__(self, w, tensors, torch, M, lo, hi, W):
        import numpy as np

        cu = w.cu_q_lens
        sub = W.Workload(f"{w.name} [{lo}:{hi}]", w.dtype, w.num_q_heads, w.num_kv_heads, w.head_dim, w.page_size,
                         w.num_pages, w.value_scale, w.seq_lens[lo:hi].copy(), w.q_lens[lo:hi].copy(),
                         np.ascontiguousarray(w.block_tables[lo:hi]), w.seed)
        t = dict(tensors, q=tensors["q"][:, int(cu[lo]):int(cu[hi])],
                 block_tables=tensors["block_tables"][lo:hi].contiguous(), seq_lens=tensors["seq_lens"][lo:hi].contiguous(),
                 cu_q_lens=torch.from_numpy(sub.cu_q_lens).cuda())
        super().__init__(sub, t, torch, M)


def measure_mixed(W, M, torch, steps, warmup):
    """One scheduler step's batch (63 decodes at 8K + a 256-token chunk on a 2K prefix, Llama-3-8B shape, F16):
    the call planned for its longest query (no host hints), the call routed per sequence class (host copies of
    the lengths), its two parts timed alone on the same tensors, and the two parts issued as separate calls
    back to back inside one timed step (parts_back_to_back: the same kernels in the same order as the routed
    call, so that the decode kernel follows a prefill as it does there; a decode kernel that follows
    decodes only runs about 9 us faster).  The routed call and the parts back to back are timed in
    alternation, three rounds each, and the no-hints call (about a millisecond of prefill kernel per step)
    last, so that no case runs right after a heavier one that the other does not follow."""
    w = W.llama3_8b_mixed_decode_prefill_f16()
    t = W.device_tensors(w, None)
    n_dec = int((w.q_lens == 1).sum())
    res = dict(workload=w.name, bytes=w.algorithmic_bytes(), flops=w.flops())
    dec = SliceRunner(w, t, torch, M, 0, n_dec, W)
    pre = SliceRunner(w, t, torch, M, n_dec, w.num_seqs, W)

    class BackToBack:
        def step(self):
            dec.step()
            pre.step()

    runners = dict(decodes_alone=dec, prefill_alone=pre, host_hints=Runner(w, t, torch, M, host_hints=True),
                   parts_back_to_back=BackToBack(), no_hints=Runner(w, t, torch, M))
    samples = {key: [] for key in runners}
    for key in ["decodes_alone", "prefill_alone"] + ["host_hints", "parts_back_to_back"] * 3 + ["no_hints"]:
        _, per = time_steps(runners[key], torch, steps, warmup)
        samples[key] += per
    for key, per in samples.items():
        per.sort()
        res[key + "_us"] = round(per[len(per) // 2], 2)
    del runners, dec, pre
    res["sum_of_parts_us"] = round(res["decodes_alone_us"] + res["prefill_alone_us"], 2)
    res["host_hints_gbs"] = round(w.algorithmic_bytes() / (res["host_hints_us"] * 1e-6) / 1e9, 1)
    res["hbm_frac"] = round(res["host_hints_gbs"] / HBM_PEAK_GBS, 4)
    del t
    torch.cuda.empty_cache()
    return res


def measure_page_sizes(W, M, torch, steps, warmup):
    """Configs 3 and 4 in pages of other sizes (README.md:175-176 lets the runner pick any): multiples of 16
    are read in place, and so are 8- and 5-token pages by the decode call and 8-token pages by the prefill
    call; the prefill call repacks 5-token pages into 16-token pages in the workspace first (a K/V copy
    inside every call)."""
    res = {}
    for cfg, sizes in ((3, (32, 48, 8, 5)), (4, (48, 8, 5))):
        for ps in sizes:
            log(f"[bench] config {cfg} in {ps}-token pages")
            res[f"{cfg}/{ps}"] = measure(W, M, torch, lambda: W.repaged(W.CONFIGS[cfg](), ps), steps, warmup)
    # The mixed step (63 decodes of 8,192 tokens + a 256-token chunk on 2,048): in 8-token pages both launches
    # read in place, in 5-token pages the whole batch is repacked first.
    for ps in (8, 5):
        log(f"[bench] mixed decode + prefill step in {ps}-token pages")
        res[f"mixed/{ps}"] = measure(W, M, torch, lambda: W.repaged(W.llama3_8b_mixed_decode_prefill_f16(), ps),
                                     steps, warmup)
    return res


DECODE_MAP = [(4, 2048), (16, 2048), (64, 2048), (16, 8192), (32, 4096), (64, 8192), (128, 2048), (128, 8192)]


def measure_decode_map(W, M, torch, steps, warmup):
    """Ragged against uniform decode at about equal bytes (Llama-3-8B shape, F16): for each (batch, ctx), the
    batch at ctx tokens each and the batch with lengths U[ctx/4, 7 ctx/4]; GB/s on each batch's own bytes."""
    rows = []
    for batch, ctx in DECODE_MAP:
        row = dict(batch=batch, ctx=ctx)
        for ragged in (False, True):
            w = W.llama3_8b_decode_map_f16(batch, ctx, ragged)
            t = W.device_tensors(w, None)
            _, per = time_steps(Runner(w, t, torch, M, host_hints=True), torch, steps, warmup)
            med = per[len(per) // 2]
            key = "ragged" if ragged else "uniform"
            row[key + "_us"] = round(med, 2)
            row[key + "_gbs"] = round(w.algorithmic_bytes() / (med * 1e-6) / 1e9, 1)
            del t
            torch.cuda.empty_cache()
        row["ragged_over_uniform"] = round(row["ragged_gbs"] / row["uniform_gbs"], 3)
        log(f"[bench] decode map b{batch} ctx{ctx}: uniform {row['uniform_gbs']} GB/s, ragged {row['ragged_gbs']} "
            f"GB/s ({row['ragged_over_uniform']:.0%})")
        rows.append(row)
    return rows


HEAD_DIMS = (32, 64, 96, 128, 160, 192, 224, 256)


def measure_head_dims(W, M, torch, steps, warmup):
    """The headline decode shape (64 x 8192 tokens, 32 Q / 8 KV heads, F16) and the Qwen2-7B chunked-prefill shape
    at every supported head dimension: 64 and 128 take the planner's full set of plans (the prefill kernel for the
    chunk), the others the split-context kernel with its merge pass."""
    res = {}
    for d in HEAD_DIMS:
        log(f"[bench] decode and prefill chunk at head_dim {d}")
        res[str(d)] = dict(decode=measure(W, M, torch, lambda: W.decode_b64_8k_head_dim_f16(d), steps, warmup),
                           prefill=measure(W, M, torch, lambda: W.chunked_prefill_head_dim_f16(d), steps, warmup))
    return res


RAGGED_PAGES = [(64, 2048), (32, 4096), (64, 8192), (128, 2048)]


def measure_ragged_pages(W, M, torch, steps, warmup):
    """Ragged decode batches (Llama-3-8B shape, F16, lengths U[ctx/4, 7 ctx/4]) in 16-, 8- and 5-token pages, the
    smaller ones read in place (token pages).  Run once as is and once with MVR_ATTN_DENSE_RAGGED=false to
    compare the dense layout with slot == partition."""
    res = {}
    for batch, ctx in RAGGED_PAGES:
        for ps in (16, 8, 5):
            log(f"[bench] ragged {batch} x U[{ctx // 4},{7 * ctx // 4}] in {ps}-token pages")
            fn = (lambda b=batch, c=ctx, ps=ps: W.repaged(W.llama3_8b_decode_map_f16(b, c, True), ps)) if ps != 16 \
                else (lambda b=batch, c=ctx: W.llama3_8b_decode_map_f16(b, c, True))
            res[f"{batch}x{ctx}r/p{ps}"] = measure(W, M, torch, fn, steps, warmup)
    return res


def measure_append(W, M, torch, cfg, steps, warmup):
    w = W.CONFIGS[cfg]()
    t = W.device_tensors(w, None)
    r = AppendRunner(w, t, torch, M, W)
    wall, per = time_steps(r, torch, steps, warmup)
    med = per[len(per) // 2]
    res = dict(workload=f"rope+append of the new tokens of {w.name} ({w.total_q} tokens)",
               us_per_step_median=round(med, 2), bytes=r.bytes,
               eff_gbs=round(r.bytes / (med * 1e-6) / 1e9, 1), hbm_frac=round(r.bytes / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
    del t, r
    torch.cuda.empty_cache()
    return res


class GatherRunner:
    """mvr_reconstruct_contiguous of one request's K: `tokens` tokens of the Llama-3-8B shape (8 KV heads, D 128) in
    16-token pages in random order, into a preallocated [1, 8, tokens, 128] tensor."""

    def __init__(self, torch, M, dtype, tokens):
        import numpy as np
        self.lib = M.load_library()
        self.tokens = tokens
        self.pages = (tokens + 15) // 16
        tdt = torch.float16 if dtype == "f16" else torch.float32
        self.pool = torch.randn((self.pages, 1, 8, 16, 128), dtype=tdt, device="cuda")
        perm = np.random.default_rng(7).permutation(self.pages).astype(np.int32)
        self.ids = torch.from_numpy(perm).cuda()
        self.out = torch.empty((1, 8, tokens, 128), dtype=tdt, device="cuda")
        self.code = M.dtype_code(self.pool)
        self.stream = torch.cuda.current_stream().cuda_stream
        self.bytes = 2 * self.out.numel() * self.out.element_size()

    def step(self):
        rc = self.lib.mvr_reconstruct_contiguous(self.code, self.pool.data_ptr(), self.pages, 8, 16, 128,
                                                 self.ids.data_ptr(), self.pages, self.tokens, self.out.data_ptr(),
                                                 self.stream)
        assert rc == 0, rc


def measure_gather(M, torch, steps, warmup):
    """The gather-to-contiguous entry point on one request's K (read + written bytes)."""
    res = {}
    for dtype in ("f16", "f32"):
        for tokens in (8192, 32768):
            r = GatherRunner(torch, M, dtype, tokens)
            _, per = time_steps(r, torch, steps, warmup)
            med = per[len(per) // 2]
            res[f"{dtype}/{tokens}"] = dict(
                workload=f"reconstruct_contiguous of one {tokens}-token request's K, 8 KV heads, D 128, {dtype}",
                us_per_step_median=round(med, 2), bytes=r.bytes, eff_gbs=round(r.bytes / (med * 1e-6) / 1e9, 1),
                hbm_frac=round(r.bytes / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
            del r
            torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 device copies of 1 GiB (a plain copy kernel of known size, for HBM counters)")
    ap.add_argument("--only-config", type=int, default=0, choices=(0, 1, 2, 4, 5),
                    help="time only this one of the other workloads and print its result (for profiling one kernel)")
    ap.add_argument("--only-mixed", action="store_true", help="time only the mixed decode + prefill batch")
    ap.add_argument("--page-sizes", action="store_true", help="time only configs 3 and 4 in other page sizes")
    ap.add_argument("--decode-map", action="store_true",
                    help="time only ragged against uniform decode batches of about equal bytes (Llama-3-8B, F16)")
    ap.add_argument("--f32", action="store_true", help="with --only-config 4: the same chunked prefill in F32")
    ap.add_argument("--only-fresh", action="store_true",
                    help="time only the Qwen2-7B fresh 8,192-token prompt (F16 prefill, one call)")
    ap.add_argument("--head-dims", action="store_true",
                    help="time only the headline decode shape at every supported head dimension")
    ap.add_argument("--ragged-pages", action="store_true",
                    help="time only ragged decode batches in 16-, 8- and 5-token pages")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {a.gpus} is not supported: the attention path runs on one "
              "GPU per call (a multi-GPU deployment shards sequences or KV heads across GPUs, each GPU running "
              "its own share)", file=sys.stderr)
        sys.exit(2)

    import torch

    import mvr_attn as M
    import workloads as W

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    M.load_library()
    if a.only_mixed:
        print(json.dumps({"mixed": measure_mixed(W, M, torch, a.steps, a.warmup)}), flush=True)
        return
    if a.page_sizes:
        print(json.dumps({"page_sizes": measure_page_sizes(W, M, torch, a.steps, a.warmup)}), flush=True)
        return
    if a.decode_map:
        print(json.dumps({"decode_map": measure_decode_map(W, M, torch, a.steps, a.warmup)}), flush=True)
        return
    if a.head_dims:
        print(json.dumps({"head_dims": measure_head_dims(W, M, torch, a.steps, a.warmup)}), flush=True)
        return
    if a.ragged_pages:
        print(json.dumps({"ragged_pages": measure_ragged_pages(W, M, torch, a.steps, a.warmup)}), flush=True)
        return
    if a.only_fresh:
        log("[bench] Qwen2-7B fresh 8,192-token prompt only")
        res = measure(W, M, torch, lambda: W.fresh_prompt_f16("qwen2-7b", 8192), a.steps, a.warmup)
        print(json.dumps({"fresh_prompt": {"qwen2-7b 1x8192": res}, "steps": a.steps, "warmup": a.warmup}), flush=True)
        return
    if a.f32 and a.only_config != 4:
        print("--f32 goes with --only-config 4", file=sys.stderr)
        sys.exit(2)
    if a.only_config:
        log(f"[bench] config {a.only_config} only{' (F32)' if a.f32 else ''}")
        cfg = (lambda: W.qwen2_7b_chunked_prefill_f16("f32")) if a.f32 else a.only_config
        res = measure(W, M, torch, cfg, a.steps, a.warmup)
        print(json.dumps({"config": a.only_config, "steps": a.steps, "warmup": a.warmup, **res}), flush=True)
        return
    headline_cfg = 3
    w = W.CONFIGS[headline_cfg]()
    log(f"[bench] headline: {w.name}")
    t = W.device_tensors(w, None)
    r = Runner(w, t, torch, M)
    wall, per = time_steps(r, torch, a.steps, a.warmup)
    med = per[len(per) // 2]
    mean = sum(per) / len(per)
    alg = w.algorithmic_bytes()
    value = alg / (mean * 1e-6) / 1e9
    log(f"[bench] headline median {med:.1f} us, mean {mean:.1f} us, {value:.0f} GB/s")
    del t, r
    torch.cuda.empty_cache()
    if a.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()

    traffic, traffic_sha = None, None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("bytes_per_launch:"):
                    traffic = int(line.split(":")[1])
                elif line.startswith("source_sha256:"):
                    traffic_sha = line.split(":")[1].strip()
    if traffic is not None and traffic_sha != traffic_source_sha256():
        log("[bench] the HBM traffic figure was measured on other kernel sources: not reported")
        traffic = None

    result = {
        "metric": "decode attention us/step + effective KV-read GB/s (% HBM peak), 1 MI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(mean / 1e3, 4),
        "us_per_step": round(mean, 2),
        "us_per_step_median": round(med, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1)*0.3 values, seeded page permutation)",
        "config": dict(w.describe(), workload="llama3-8b-shape paged decode attention, batch 64 x 8192 ctx, "
                                             "32q/8kv heads, head_dim 128, 16-token pages, f16"),
        "roofline": {
            "bound": "hbm",
            "achieved": round(value, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "timed": "mean duration of the whole attention call between HIP events recorded on the launch stream "
                     "(one launch of paged_attention_kernel, whose 4 context partitions per (sequence, KV head) "
                     "merge in LDS); the rocprofv3 kernel-trace summary in profiles/ lists its average, which "
                     "this mean should match",
        },
    }
    if not a.only_headline:
        per_cfg = {}
        for cfg in (1, 2, 4, 5):
            log(f"[bench] config {cfg}")
            per_cfg[str(cfg)] = measure(W, M, torch, cfg, max(20, a.steps // 2), a.warmup)
        result["configs"] = per_cfg
        log("[bench] F32 (the activation dtype the reference's GPU backends force) at configs 3 and 4")
        result["f32"] = {
            "3": measure(W, M, torch, lambda: W.llama3_8b_decode_b64_8k_f16(64, "f32"), max(20, a.steps // 2), a.warmup),
            "4": measure(W, M, torch, lambda: W.qwen2_7b_chunked_prefill_f16("f32"), max(20, a.steps // 2), a.warmup),
        }
        log("[bench] fresh prompts (prefill with nothing cached)")
        result["fresh_prompt"] = {
            "llama3-8b 1x2048": measure(W, M, torch, lambda: W.fresh_prompt_f16("llama3-8b", 2048),
                                        max(20, a.steps // 2), a.warmup),
            "qwen2-7b 1x8192": measure(W, M, torch, lambda: W.fresh_prompt_f16("qwen2-7b", 8192),
                                       max(20, a.steps // 2), a.warmup),
        }
        log("[bench] mixed decode + prefill batch")
        result["mixed"] = measure_mixed(W, M, torch, max(20, a.steps // 2), a.warmup)
        log("[bench] config 5 through cascade attention")
        result["cascade"] = {"5": measure_cascade(W, M, torch, 5, max(20, a.steps // 2), a.warmup)}
        log("[bench] shared-prompt decode, cascade and plain")
        result["cascade"]["shared_prompt"] = measure_cascade(W, M, torch, W.llama3_8b_shared_prompt_decode_f16,
                                                             max(20, a.steps // 2), a.warmup, with_plain=True)
        result["page_sizes"] = measure_page_sizes(W, M, torch, max(20, a.steps // 2), a.warmup)
        result["rope_append"] = {}
        for cfg in (3, 4):
            log(f"[bench] rope+append, config {cfg}")
            result["rope_append"][str(cfg)] = measure_append(W, M, torch, cfg, max(20, a.steps // 2), a.warmup)
        log("[bench] gather to contiguous")
        result["gather"] = measure_gather(M, torch, max(20, a.steps // 2), a.warmup)
    if not a.skip_cpu:
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline(W)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
