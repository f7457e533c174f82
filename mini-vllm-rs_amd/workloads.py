"""Seeded synthetic page-wise attention workloads.

Five shapes: Qwen2-0.5B decode (F32 and batched F16), Llama-3-8B batch-64 x 8K
decode, Qwen2-7B chunked prefill and Llama-3-8B speculative verification with
shared prefix pages; and a sixth for cascade attention, a Llama-3-8B decode
batch whose sequences share one long prompt prefix.  Block tables, lengths and values are derived from a seed
so the GPU and the CPU see identical bytes: tables and lengths with numpy's
PCG64, values either with numpy (host, for parity tests) or torch's device
generator (fast, for benchmarks).

Layouts follow the reference's data contract (src/models/mod.rs:56-100):
pools [num_pages, 1, Hkv, page_size, D]; q / out [Hq, total_q, D] (the packed
[1, Hq, packed_q_len, D] layout of common.rs:268-275); block tables int32
[num_seqs, max_pages_per_seq]; seq_lens = cached_token_count (current query
included); cu_q_lens = prefix sums of q_len.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

SEED_BASE = 0x6D76720000


@dataclass
class Workload:
    name: str
    dtype: str  # "f32" | "f16"
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    num_pages: int
    value_scale: float
    seq_lens: np.ndarray       # int32 [B]
    q_lens: np.ndarray         # int32 [B]
    block_tables: np.ndarray   # int32 [B, max_pages]
    seed: int
    shared_pages: int = 0      # pages read by more than one sequence (counted once in unique bytes)
    notes: str = ""
    # Groups of consecutive sequences sharing their first pages: (first_seq, n_seqs, prefix_tokens).
    prefix_groups: List = field(default_factory=list)

    @property
    def num_seqs(self) -> int:
        return len(self.seq_lens)

    @property
    def cu_q_lens(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)

    @property
    def total_q(self) -> int:
        return int(self.q_lens.sum())

    @property
    def elem_size(self) -> int:
        return 2 if self.dtype == "f16" else 4

    @property
    def np_dtype(self):
        return np.float16 if self.dtype == "f16" else np.float32

    @property
    def max_q_len(self) -> int:
        return int(self.q_lens.max())

    @property
    def max_seq_len(self) -> int:
        return int(self.seq_lens.max())

    def kv_bytes(self) -> int:
        """Logical K+V bytes one call reads: every visible token of every sequence."""
        return int(self.seq_lens.sum()) * self.num_kv_heads * self.head_dim * self.elem_size * 2

    def unique_kv_bytes(self) -> int:
        return self.kv_bytes() - self.shared_pages * self.page_size * self.num_kv_heads * self.head_dim * \
            self.elem_size * 2

    def algorithmic_bytes(self, unique: bool = False) -> int:
        """K/V read + Q read + O written + block-table entries read."""
        kv = self.unique_kv_bytes() if unique else self.kv_bytes()
        qo = self.total_q * self.num_q_heads * self.head_dim * self.elem_size * 2
        bt = int(sum(math.ceil(int(L) / self.page_size) for L in self.seq_lens)) * 4
        return kv + qo + bt

    def flops(self) -> int:
        """2 flops per multiply-add for QK^T and PV over causally visible (query, key) pairs."""
        pairs = 0
        for L, q in zip(self.seq_lens.tolist(), self.q_lens.tolist()):
            c = L - q
            pairs += q * c + q * (q + 1) // 2
        return 4 * pairs * self.num_q_heads * self.head_dim

    def describe(self) -> Dict:
        return dict(workload=self.name, dtype=self.dtype, num_seqs=self.num_seqs, num_q_heads=self.num_q_heads,
                    num_kv_heads=self.num_kv_heads, head_dim=self.head_dim, page_size=self.page_size,
                    num_pages=self.num_pages, total_q=self.total_q, max_seq_len=self.max_seq_len,
                    sum_seq_len=int(self.seq_lens.sum()), seed=self.seed)


def _assign_pages(rng, seq_lens, page_size, num_pages):
    """Pages for each sequence drawn in order from one shuffle of the pool."""
    perm = rng.permutation(num_pages).astype(np.int32)
    need = [math.ceil(int(L) / page_size) for L in seq_lens]
    if sum(need) > num_pages:
        raise ValueError("pool too small")
    bt = np.zeros((len(seq_lens), max(need)), np.int32)
    used = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[used:used + n]
        used += n
    return bt


def qwen2_05b_decode_f32() -> Workload:
    """1 sequence, 1 query token, 14 Q / 2 KV heads, D 64, 512 tokens in 16-token pages, pool 64 pages."""
    seed = SEED_BASE + 1
    rng = np.random.default_rng(seed)
    perm = rng.permutation(64).astype(np.int32)
    return Workload("qwen2-0.5b decode f32 b1 ctx512", "f32", 14, 2, 64, 16, 64, 0.5,
                    np.array([512], np.int32), np.array([1], np.int32), perm[None, :32].copy(), seed)


def qwen2_05b_batched_decode_f16() -> Workload:
    """Batch 8, lengths U[128, 4096], 14 Q / 2 KV, D 64, pool of 4096 pages."""
    seed = SEED_BASE + 2
    rng = np.random.default_rng(seed)
    seq_lens = rng.integers(128, 4096, size=8, endpoint=True).astype(np.int32)
    bt = _assign_pages(rng, seq_lens, 16, 4096)
    return Workload("qwen2-0.5b decode f16 b8 ctxU[128,4096]", "f16", 14, 2, 64, 16, 4096, 0.5, seq_lens,
                    np.ones(8, np.int32), bt, seed)


def llama3_8b_decode_b64_8k_f16(batch: int = 64, dtype: str = "f16") -> Workload:
    """Batch 64 x 8192 tokens, 32 Q / 8 KV, D 128, pool = exact fit (32768 pages), permuted.  dtype "f32" gives the
    same shape in F32, the activation dtype the reference's GPU backends force (server/mod.rs:505-530)."""
    seed = SEED_BASE + 3
    rng = np.random.default_rng(seed)
    seq_lens = np.full(batch, 8192, np.int32)
    num_pages = batch * 512
    bt = _assign_pages(rng, seq_lens, 16, num_pages)
    return Workload(f"llama3-8b decode {dtype} b{batch} ctx8192", dtype, 32, 8, 128, 16, num_pages, 0.3, seq_lens,
                    np.ones(batch, np.int32), bt, seed)


def decode_b64_8k_head_dim_f16(head_dim: int, batch: int = 64) -> Workload:
    """The headline decode shape (batch x 8192 tokens, 32 Q / 8 KV heads, F16, 16-token pages in random order, pool
    = exact fit) at another head dimension, for timing the head dimensions besides 64 and 128."""
    seed = SEED_BASE + 17 + head_dim
    rng = np.random.default_rng(seed)
    seq_lens = np.full(batch, 8192, np.int32)
    num_pages = batch * 512
    bt = _assign_pages(rng, seq_lens, 16, num_pages)
    return Workload(f"decode f16 b{batch} ctx8192 32/8 heads D{head_dim}", "f16", 32, 8, head_dim, 16, num_pages, 0.3,
                    seq_lens, np.ones(batch, np.int32), bt, seed)


def chunked_prefill_head_dim_f16(head_dim: int) -> Workload:
    """The Qwen2-7B chunked-prefill shape (4 x 256 new tokens on 2048 cached, 28 Q / 4 KV heads, F16) at another
    head dimension."""
    w = qwen2_7b_chunked_prefill_f16()
    return Workload(f"qwen2-7b-shaped chunked prefill f16 D{head_dim}", "f16", w.num_q_heads, w.num_kv_heads, head_dim,
                    w.page_size, w.num_pages, w.value_scale, w.seq_lens, w.q_lens, w.block_tables, w.seed + head_dim)


def qwen2_7b_chunked_prefill_f16(dtype: str = "f16") -> Workload:
    """4 sequences, 2048 cached + 256 new tokens, 28 Q / 4 KV, D 128, pages in random order (dtype "f32": the same
    shape in F32)."""
    seed = SEED_BASE + 4
    rng = np.random.default_rng(seed)
    seq_lens = np.full(4, 2048 + 256, np.int32)
    num_pages = 4 * math.ceil(2304 / 16)
    bt = _assign_pages(rng, seq_lens, 16, num_pages)
    return Workload(f"qwen2-7b chunked prefill {dtype} b4 2048+256", dtype, 28, 4, 128, 16, num_pages, 0.3, seq_lens,
                    np.full(4, 256, np.int32), bt, seed)


def fresh_prompt_f16(model: str = "llama3-8b", prompt: int = 2048, num_seqs: int = 1) -> Workload:
    """Prefill of whole prompts with nothing cached (q_len = seq_len, the first chunk of a request when the
    scheduler's budget admits the prompt at once): causal self-attention over the prompt, pages in random order.
    model: "llama3-8b" (32 Q / 8 KV, D 128) or "qwen2-7b" (28 Q / 4 KV, D 128)."""
    hq, hkv = {"llama3-8b": (32, 8), "qwen2-7b": (28, 4)}[model]
    seed = SEED_BASE + 8
    rng = np.random.default_rng(seed)
    seq_lens = np.full(num_seqs, prompt, np.int32)
    num_pages = num_seqs * math.ceil(prompt / 16)
    bt = _assign_pages(rng, seq_lens, 16, num_pages)
    return Workload(f"{model} fresh prompt f16 b{num_seqs} {prompt}", "f16", hq, hkv, 128, 16, num_pages, 0.3,
                    seq_lens, np.full(num_seqs, prompt, np.int32), bt, seed)


def llama3_8b_mixed_decode_prefill_f16(num_decode: int = 63, decode_ctx: int = 8192, prefix: int = 2048,
                                       chunk: int = 256, dtype: str = "f16") -> Workload:
    """The batch one scheduler step emits (scheduler.rs:258-271): the decode requests first, one token each,
    then the prefill chunk that the remaining token budget admits.  Llama-3-8B shape (32 Q / 8 KV, D 128):
    63 decodes over 8192 cached tokens and one 256-token chunk on a 2048-token cached prefix, 16-token pages
    in random order."""
    seed = SEED_BASE + 7
    rng = np.random.default_rng(seed)
    seq_lens = np.array([decode_ctx + 1] * num_decode + [prefix + chunk], np.int32)
    q_lens = np.array([1] * num_decode + [chunk], np.int32)
    num_pages = int(sum(math.ceil(int(L) / 16) for L in seq_lens))
    bt = _assign_pages(rng, seq_lens, 16, num_pages)
    return Workload(f"llama3-8b mixed {dtype} {num_decode} decodes ctx{decode_ctx} + prefill {prefix}+{chunk}", dtype,
                    32, 8, 128, 16, num_pages, 0.3, seq_lens, q_lens, bt, seed)


def llama3_8b_decode_map_f16(batch: int, ctx: int, ragged: bool) -> Workload:
    """Llama-3-8B-shaped F16 decode (32 Q / 8 KV, D 128, one query token each) over `batch` sequences of `ctx`
    cached tokens (uniform) or of lengths drawn from U[ctx/4, 7 ctx/4] (ragged: the same mean, so about the same
    bytes), 16-token pages in random order, pool = exact fit."""
    seed = SEED_BASE + 11 + batch + ctx + int(ragged)
    rng = np.random.default_rng(seed)
    if ragged:
        seq_lens = rng.integers(ctx // 4, 7 * ctx // 4, size=batch, endpoint=True).astype(np.int32)
    else:
        seq_lens = np.full(batch, ctx, np.int32)
    num_pages = int(sum(math.ceil(int(L) / 16) for L in seq_lens))
    bt = _assign_pages(rng, seq_lens, 16, num_pages)
    kind = f"U[{ctx // 4},{7 * ctx // 4}]" if ragged else f"{ctx}"
    return Workload(f"llama3-8b decode f16 b{batch} ctx{kind}", "f16", 32, 8, 128, 16, num_pages, 0.3, seq_lens,
                    np.ones(batch, np.int32), bt, seed)


def repaged(w: Workload, page_size: int) -> Workload:
    """The same requests (lengths, query lengths, heads, dtype) stored in pages of page_size tokens in a random
    order, pool = exact fit: for timing a page size against the 16-token layout."""
    rng = np.random.default_rng(w.seed + 1000 * page_size)
    num_pages = int(sum(math.ceil(int(L) / page_size) for L in w.seq_lens))
    bt = _assign_pages(rng, w.seq_lens, page_size, num_pages)
    return Workload(f"{w.name}, {page_size}-token pages", w.dtype, w.num_q_heads, w.num_kv_heads, w.head_dim, page_size,
                    num_pages, w.value_scale, w.seq_lens.copy(), w.q_lens.copy(), bt, w.seed)


def llama3_8b_spec_verify_f16() -> Workload:
    """16 sequences verifying 5 positions; contexts U[1024, 16384]; groups of 4 share the first 1024 tokens' pages."""
    seed = SEED_BASE + 5
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1024, 16384, size=16, endpoint=True).astype(np.int32)
    q = 5
    seq_lens = (ctx + q).astype(np.int32)
    shared = 1024 // 16
    private = [math.ceil(int(L) / 16) - shared for L in seq_lens]
    num_pages = 4 * shared + sum(private)
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((16, max(p + shared for p in private)), np.int32)
    used = 0
    group_prefix = []
    for grp in range(4):
        group_prefix.append(perm[used:used + shared])
        used += shared
    for s in range(16):
        bt[s, :shared] = group_prefix[s // 4]
        bt[s, shared:shared + private[s]] = perm[used:used + private[s]]
        used += private[s]
    # Each group's prefix pages are read by 4 sequences; 3 of the 4 reads are repeats.
    return Workload("llama3-8b spec-verify f16 b16 q5 ctxU[1024,16384] shared-prefix", "f16", 32, 8, 128, 16,
                    num_pages, 0.3, seq_lens, np.full(16, q, np.int32), bt, seed, shared_pages=12 * shared,
                    prefix_groups=[(4 * g, 4, 1024) for g in range(4)])


def llama3_8b_shared_prompt_decode_f16(batch: int = 64, prompt: int = 8192, lo: int = 256, hi: int = 2048) -> Workload:
    """One decode step of `batch` sequences that share a `prompt`-token prefix (a system prompt: one set of
    physical pages, as find_longest_cached_prefix hands a cached prefix's pages to every request that
    matches it, prefix_index.rs:174-211) followed by private contexts of U[lo, hi] tokens."""
    seed = SEED_BASE + 6
    rng = np.random.default_rng(seed)
    q = 1
    seq_lens = (prompt + rng.integers(lo, hi, size=batch, endpoint=True) + q).astype(np.int32)
    shared = prompt // 16
    private = [math.ceil(int(L) / 16) - shared for L in seq_lens]
    num_pages = shared + sum(private)
    perm = rng.permutation(num_pages).astype(np.int32)
    bt = np.zeros((batch, max(p + shared for p in private)), np.int32)
    bt[:, :shared] = perm[:shared]
    used = shared
    for s in range(batch):
        bt[s, shared:shared + private[s]] = perm[used:used + private[s]]
        used += private[s]
    # The prompt's pages are read by every sequence; batch - 1 of those reads are repeats.
    return Workload(f"llama3-8b decode f16 b{batch} shared-prompt {prompt} + ctxU[{lo},{hi}]", "f16", 32, 8, 128, 16,
                    num_pages, 0.3, seq_lens, np.full(batch, q, np.int32), bt, seed,
                    shared_pages=(batch - 1) * shared, prefix_groups=[(0, batch, prompt)])


CONFIGS = {
    1: qwen2_05b_decode_f32,
    2: qwen2_05b_batched_decode_f16,
    3: llama3_8b_decode_b64_8k_f16,
    4: qwen2_7b_chunked_prefill_f16,
    5: llama3_8b_spec_verify_f16,
}


def rope_tables(head_dim: int, freq_base: float, context_len: int, dtype=np.float16):
    """cos / sin tables [context_len, head_dim/2] as precompute_rotary_embedding_frequencies builds them
    (src/models/backends/common.rs:558-577): theta_i = 1 / base^(2i/D) in f32, angle = position * theta_i
    in f32, cos and sin in f32, then cast to the activation dtype."""
    i = np.arange(0, head_dim, 2, dtype=np.float32)
    theta = np.float32(1.0) / np.power(np.float32(freq_base), i / np.float32(head_dim), dtype=np.float32)
    angle = np.arange(context_len, dtype=np.float32)[:, None] * theta[None, :]
    return np.cos(angle).astype(dtype), np.sin(angle).astype(dtype)


def host_values(w: Workload, chunk: int = 1 << 26):
    """(q, key_pool, value_pool) as numpy arrays in the workload dtype, N(0,1)*scale, from numpy's PCG64."""
    rng = np.random.default_rng(w.seed ^ 0x5EED)
    shape_pool = (w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim)

    def normal(shape):
        out = np.empty(shape, w.np_dtype)
        flat = out.reshape(-1)
        for s in range(0, flat.size, chunk):
            n = min(chunk, flat.size - s)
            flat[s:s + n] = (rng.standard_normal(n, dtype=np.float32) * np.float32(w.value_scale)).astype(w.np_dtype)
        return out

    q = normal((w.num_q_heads, w.total_q, w.head_dim))
    k = normal(shape_pool)
    v = normal(shape_pool)
    return q, k, v


def device_tensors(w: Workload, values: Optional[tuple] = None, device: str = "cuda", seed: Optional[int] = None):
    """Torch tensors on the device.  values=None draws them on the device with torch's generator."""
    import torch

    tdt = torch.float16 if w.dtype == "f16" else torch.float32
    if values is None:
        g = torch.Generator(device=device)
        g.manual_seed(w.seed if seed is None else seed)
        shape_pool = (w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim)

        def normal(shape):
            t = torch.empty(shape, dtype=tdt, device=device)
            t.normal_(0.0, w.value_scale, generator=g)
            return t

        q, k, v = normal((w.num_q_heads, w.total_q, w.head_dim)), normal(shape_pool), normal(shape_pool)
    else:
        q, k, v = (torch.from_numpy(np.ascontiguousarray(x)).to(device) for x in values)
    bt = torch.from_numpy(w.block_tables).to(device)
    sl = torch.from_numpy(w.seq_lens).to(device)
    cu = torch.from_numpy(w.cu_q_lens).to(device)
    return dict(q=q, key_pool=k, value_pool=v, block_tables=bt, seq_lens=sl, cu_q_lens=cu)


def cascade_tables(w: Workload):
    """Host arrays describing w.prefix_groups for cascade attention: group_cu_q_lens, group_prefix_lens,
    group_block_tables, seq_prefix_lens (int32)."""
    cu = w.cu_q_lens
    groups = w.prefix_groups
    gcu = np.array([cu[g[0]] for g in groups] + [cu[groups[-1][0] + groups[-1][1]]], np.int32)
    gpre = np.array([g[2] for g in groups], np.int32)
    gbt = np.stack([w.block_tables[g[0]] for g in groups]).astype(np.int32)
    spre = np.zeros(w.num_seqs, np.int32)
    for first, n, pre in groups:
        spre[first:first + n] = pre
    return gcu, gpre, gbt, spre
