"""Seeded synthetic inputs of the verify path (the five benchmark configurations).

1. CPU plumbing: B=4, ctx in [64,256], k=4 (5 query tokens, causal), 8/2 heads,
   D=64, page 16, fp32; greedy acceptance over V=1000.
2. Llama-3-8B verify: B=64, ctx in [1024,4096], k=4, 32/8 heads, D=128, page 16,
   bf16, values N(0,1)*0.5, plus the append of the 5 new K/V rows per request.
3. MagicDec long context: B=32, ctx in [32768,65536]; (a) 1 query over a 64-sink +
   512-window view, (b) 5 causal queries over the full context.
4. EAGLE tree: B=32, ctx in [2048,8192], a 32-node draft tree per request (parent
   drawn among nodes of depth < 6 with < 4 children), ancestor bitmask.
5. Stochastic acceptance: B=128, k=5, V=128256, T=1; target logits N(0, 2^2), draft
   logits = target + N(0, 0.5^2), draft tokens drawn from the draft softmax.
Pages are a seeded random permutation; kv lengths already include the appended
draft tokens (the page table is updated before the layer loop).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from .masks import tree_mask_words


@dataclass
class VerifyBatch:
    qo_indptr: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    q: torch.Tensor          # [nnz, Hq, D]
    cache: torch.Tensor      # [P, 2, ps, Hkv, D]
    k_new: torch.Tensor      # [nnz, Hkv, D] rows appended at the tail of each request
    v_new: torch.Tensor
    ctx: np.ndarray          # kv tokens before the append
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    mask_words: Optional[np.ndarray] = None  # tree mode, one word per query token
    tree_depth: Optional[np.ndarray] = None
    sink: int = 0
    window: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def kv_lens(self) -> np.ndarray:
        n = np.diff(self.kv_indptr.cpu().numpy().astype(np.int64))
        last = self.kv_last_page_len.cpu().numpy().astype(np.int64)
        return np.where(n > 0, (n - 1) * self.page_size + last, 0)

    def to(self, device) -> "VerifyBatch":
        kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return VerifyBatch(**kw)


def random_tree_parents(n: int, rng: np.random.Generator, max_depth: int = 6,
                        max_children: int = 4) -> np.ndarray:
    parents = np.full(n, -1, dtype=np.int64)
    depth = np.zeros(n, dtype=np.int64)
    children = np.zeros(n, dtype=np.int64)
    for i in range(1, n):
        cand = [j for j in range(i) if depth[j] < max_depth and children[j] < max_children]
        p = int(rng.choice(cand))
        parents[i] = p
        depth[i] = depth[p] + 1
        children[p] += 1
    return parents


def make_verify_batch(batch: int, ctx_lo: int, ctx_hi: int, qo_len: int, num_qo_heads: int,
                      num_kv_heads: int, head_dim: int, page_size: int = 16,
                      dtype: torch.dtype = torch.bfloat16, scale: float = 1.0, seed: int = 0,
                      device="cpu", tree_nodes: int = 0, extra_pages: int = 0,
                      qo_lens: Optional[np.ndarray] = None, ctx: Optional[np.ndarray] = None,
                      page_order: str = "random") -> VerifyBatch:
    """Random paged batch; values drawn with a torch generator on `device`."""
    rng = np.random.default_rng(seed)
    if ctx is None:
        ctx = rng.integers(ctx_lo, ctx_hi + 1, size=batch).astype(np.int64)
    if qo_lens is None:
        qo_lens = np.full(batch, qo_len, dtype=np.int64)
    kv = ctx + qo_lens
    pages = np.maximum(1, (kv + page_size - 1) // page_size)
    last = np.where(kv > 0, (kv - 1) % page_size + 1, 0)
    kv_indptr = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    total_pages = int(kv_indptr[-1]) + extra_pages
    perm = rng.permutation(total_pages).astype(np.int32)[: int(kv_indptr[-1])]
    if page_order == "sequential":
        perm = np.arange(int(kv_indptr[-1]), dtype=np.int32)
    qo_indptr = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    nnz = int(qo_indptr[-1])
    gen = torch.Generator(device=device).manual_seed(seed)
    dev = torch.device(device)

    def randn(*shape):
        if dev.type == "cpu" and dtype != torch.float32:
            return (torch.randn(shape, generator=gen, dtype=torch.float32) * scale).to(dtype)
        return torch.randn(shape, generator=gen, dtype=dtype, device=dev) * scale

    q = randn(nnz, num_qo_heads, head_dim)
    cache = randn(total_pages, 2, page_size, num_kv_heads, head_dim)
    k_new = randn(nnz, num_kv_heads, head_dim)
    v_new = randn(nnz, num_kv_heads, head_dim)
    words = depth = None
    if tree_nodes:
        words = np.zeros(nnz, dtype=np.uint32)
        depth = np.zeros(nnz, dtype=np.int64)
        for b in range(batch):
            par = random_tree_parents(int(qo_lens[b]), rng)
            w, d = tree_mask_words(par)
            words[qo_indptr[b]:qo_indptr[b + 1]] = w
            depth[qo_indptr[b]:qo_indptr[b + 1]] = d
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)
    return VerifyBatch(i32(qo_indptr), i32(kv_indptr), i32(perm), i32(last), q, cache, k_new,
                       v_new, ctx, num_qo_heads, num_kv_heads, head_dim, page_size,
                       mask_words=words, tree_depth=depth)


# ---- the benchmark configurations -------------------------------------------------

def config1(device="cpu", dtype=torch.float32) -> VerifyBatch:
    return make_verify_batch(4, 64, 256, 5, 8, 2, 64, 16, dtype=dtype, seed=1001, device=device)


def config2(device="cpu", seed: int = 1002, page_order: str = "random") -> VerifyBatch:
    return make_verify_batch(64, 1024, 4096, 5, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5,
                             seed=seed, device=device, page_order=page_order)


def config3(device="cpu", seed: int = 1003, batch: int = 32) -> VerifyBatch:
    b = make_verify_batch(batch, 32768, 65536, 5, 32, 8, 128, 16, dtype=torch.bfloat16,
                          scale=0.5, seed=seed, device=device)
    b.sink, b.window = 64, 512
    return b


def config4(device="cpu", seed: int = 1004, batch: int = 32) -> VerifyBatch:
    return make_verify_batch(batch, 2048, 8192, 32, 32, 8, 128, 16, dtype=torch.bfloat16,
                             scale=0.5, seed=seed, device=device, tree_nodes=32)


@dataclass
class AcceptCase:
    target_logits: torch.Tensor  # [B, k+1, V]
    draft_logits: Optional[torch.Tensor]  # [B, k, V]
    draft_tokens: torch.Tensor   # [B, k] int64
    uniforms: torch.Tensor       # [B, k+1] fp32
    temperature: float = 1.0
    eos_token_id: int = -1


def greedy_case(B: int = 4, k: int = 4, V: int = 1000, p_match: float = 0.7, seed: int = 1001,
                dtype=torch.float32, device="cpu") -> AcceptCase:
    """Target logits N(0,1); draft_i = target argmax with probability p_match, else uniform."""
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn((B, k + 1, V), generator=gen).to(dtype)
    am = logits.float().argmax(-1)[:, :k]
    rnd = torch.randint(0, V, (B, k), generator=gen)
    keep = torch.rand((B, k), generator=gen) < p_match
    draft = torch.where(keep, am, rnd).to(torch.int64)
    u = torch.rand((B, k + 1), generator=gen)
    return AcceptCase(logits.to(device), None, draft.to(device), u.to(device))


def stochastic_case(B: int = 128, k: int = 5, V: int = 128256, sigma: float = 2.0,
                    noise: float = 0.5, temperature: float = 1.0, seed: int = 1005,
                    dtype=torch.bfloat16, device="cpu") -> AcceptCase:
    """Config 5.  Values are drawn on `device`; draft tokens by inverse CDF of the
    draft softmax (float64 on the host) with seeded uniforms."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    target = (torch.randn((B, k + 1, V), generator=gen, device=dev) * sigma)
    draft = target[:, :k, :] + torch.randn((B, k, V), generator=gen, device=dev) * noise
    target = target.to(dtype)
    draft = draft.to(dtype)
    rng = np.random.default_rng(seed)
    d64 = draft.double() / temperature
    probs = torch.softmax(d64, dim=-1)
    cdf = torch.cumsum(probs, dim=-1)
    uu = torch.from_numpy(rng.random((B, k, 1))).to(dev)
    tok = torch.searchsorted(cdf, uu * cdf[..., -1:]).clamp_max(V - 1)[..., 0].to(torch.int64)
    u = torch.from_numpy(rng.random((B, k + 1)).astype(np.float32)).to(dev)
    return AcceptCase(target, draft, tok, u, temperature)
