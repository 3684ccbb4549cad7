"""Producers of the verify-step attention masks and position ids.

* ``mtp_attn_mask_and_position_ids`` — the (k+1)^2 interleaved MTP pattern of
  batchspec/backends/mtp_engine.py:172-208: row i (group g_i = i // (k+1), slot
  r_i = i % (k+1)) sees column j iff (r_j == 0 and j <= i) or
  (g_i == g_j and 1 <= r_j <= r_i); position_ids[i] = g_i + r_i.
* ``mtp_verify_custom_mask`` — the flattened per-request mask
  cat(ones(S, cachelen_b), common_mask) of mtp_engine.py:410-417.
* ``tree_mask_words`` — ancestor-or-self bit words of a draft tree given by a parent
  array (EAGLE-style verification), one uint32 per node, bit j = node j.
* ``mtp_parents`` / ``tree_masks`` / ``MTPMaskMixin`` — the same words and the position
  ids built on the GPU from parent arrays (the MTP layout is a tree), so the verify
  step needs no host mask (replacing mtp_engine.py:172-208 and :410-417).
The bit words are what ``BatchPrefillWithPagedKVCacheWrapper.plan(tree_mask_words=...)``
consumes; they replace the O(qo * kv) bool mask.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from ._util import require_gpu, stream_of


def mtp_attn_mask_and_position_ids(draft_length: int, device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    S = (draft_length + 1) ** 2
    idx = torch.arange(S, device=device)
    g = idx // (draft_length + 1)
    r = idx % (draft_length + 1)
    regular = (r[None, :] == 0) & (idx[None, :] <= idx[:, None])
    same_group = (g[:, None] == g[None, :]) & (r[None, :] > 0) & (r[None, :] <= r[:, None])
    return regular | same_group, (g + r).to(torch.long)


def mtp_verify_custom_mask(cachelens: Sequence[int], draft_length: int, device=None) -> torch.Tensor:
    common, _ = mtp_attn_mask_and_position_ids(draft_length, device)
    S = common.shape[0]
    parts = [torch.cat((torch.ones((S, int(c)), dtype=torch.bool, device=device), common), dim=-1)
             .flatten() for c in cachelens]
    return torch.cat(parts) if parts else torch.zeros(0, dtype=torch.bool, device=device)


def mask_to_words(mask: torch.Tensor) -> np.ndarray:
    """[n, n] bool (n <= 32) -> uint32 per row, bit j = mask[i, j]."""
    m = mask.detach().to("cpu", torch.bool).numpy()
    n = m.shape[1]
    if n > 32:
        raise ValueError("at most 32 columns fit a word")
    return (m.astype(np.uint64) << np.arange(n, dtype=np.uint64)).sum(axis=1).astype(np.uint32)


def tree_mask_words(parents: Sequence[int]) -> Tuple[np.ndarray, np.ndarray]:
    """Ancestor-or-self words and depths of a tree given parent[i] < i (-1 = root
    attached to the prefix).  Returns (words uint32 [n], depth int64 [n])."""
    n = len(parents)
    if n > 32:
        raise ValueError("at most 32 tree nodes")
    words = np.zeros(n, dtype=np.uint32)
    depth = np.zeros(n, dtype=np.int64)
    for i, p in enumerate(parents):
        p = int(p)
        if p >= i:
            raise ValueError("parent[i] must precede i")
        if p < 0:
            words[i] = np.uint32(1 << i)
            depth[i] = 0
        else:
            words[i] = words[p] | np.uint32(1 << i)
            depth[i] = depth[p] + 1
    return words, depth


def mtp_parents(draft_length: int) -> np.ndarray:
    """Parent array (int32 [(k+1)^2]) of the MTP layout of mtp_engine.py:172-208 read as a
    tree: regular token x_g (index g(k+1)) hangs off x_{g-1} (x_0 off the cached prefix,
    -1) and mask token m_r of group g off the token before it (m_1 off x_g).  Its
    ancestor-or-self relation is the MTP mask and its depths g + r are the position ids."""
    k1 = draft_length + 1
    S = k1 * k1
    par = np.empty(S, dtype=np.int32)
    for i in range(S):
        g, r = divmod(i, k1)
        par[i] = (i - 1) if r > 0 else ((g - 1) * k1 if g > 0 else -1)
    return par


def tree_masks(parents: torch.Tensor, cachelens: Optional[torch.Tensor] = None,
               batch: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Tree-mask words and positions on the GPU, with no host round trip.

    parents: int32 [B, n] per request, or [n] shared by ``batch`` requests (parent[i] < i,
    -1 for a node hanging off the cached prefix; n <= 32).  cachelens: [B] (any int
    dtype) or None (0).  Returns (words int32 [B, n], the ``tree_mask_words`` of
    ``BatchPrefillWithPagedKVCacheWrapper.plan``; positions int64 [B, n] = cachelen +
    depth)."""
    dev = require_gpu("tree_masks", parents, cachelens)
    par = parents.to(torch.int32).contiguous()
    if par.dim() == 1:
        n = par.shape[0]
        B = int(batch) if batch is not None else (cachelens.shape[0] if cachelens is not None else 1)
        stride = 0
    elif par.dim() == 2:
        B, n = par.shape
        stride = n
    else:
        raise ValueError("parents must be [n] or [B, n]")
    if n > 32:
        raise ValueError("at most 32 draft tokens per request")
    cl = None
    if cachelens is not None:
        if cachelens.numel() != B:
            raise ValueError(f"cachelens must have {B} entries")
        cl = cachelens.to(torch.int32).contiguous()
    words = torch.empty((B, n), dtype=torch.int32, device=dev)
    pos = torch.empty((B, n), dtype=torch.int64, device=dev)
    rc = _lib.load().bsx_tree_masks(par.data_ptr(), stride, n, _lib.ptr(cl), B, words.data_ptr(),
                                    pos.data_ptr(), stream_of(dev))
    _lib.check(rc, "tree_masks")
    return words, pos


class MTPMaskMixin:
    """MTPEngine's verify-step mask without the host loop: ``pre_draft_and_verify``
    (mtp_engine.py:399-432) plans with device-built tree words of the MTP layout
    instead of the concatenated bool mask, and ``verify_position_ids()`` gives
    cachelens[:, None] + common_position_ids (mtp_engine.py:381) from the same kernel.
    Reads ``draft_length``, ``device``, ``cachelens``, ``qo_indptr``, the page-table
    buffers, ``attn_wrappers``, ``model.config`` and ``dtype`` like the reference."""

    def _setup_common_attn_mask_and_position_ids(self):
        m, pos = mtp_attn_mask_and_position_ids(self.draft_length, self.device)
        self.common_attn_mask = m
        self.common_position_ids = pos
        self.common_parents = torch.from_numpy(mtp_parents(self.draft_length)).to(self.device)

    def verify_position_ids(self) -> torch.Tensor:
        _, pos = tree_masks(self.common_parents, self.cachelens)
        return pos.flatten()

    def pre_draft_and_verify(self, bsz: int, dec_len: int):
        words, _ = tree_masks(self.common_parents, self.cachelens[:bsz])
        self.insert_kv(dec_len)
        cfg = self.model.config
        self.attn_wrappers["draft_and_verify"].plan(
            qo_indptr=self.qo_indptr * dec_len,
            paged_kv_indptr=self.paged_kv_indptr,
            paged_kv_indices=self.paged_kv_indices,
            paged_kv_last_page_len=self.paged_kv_last_page_len,
            num_qo_heads=cfg.n_head,
            num_kv_heads=cfg.n_local_heads,
            head_dim_qk=cfg.head_dim,
            page_size=self.page_size,
            q_data_type=self.dtype,
            causal=False,
            tree_mask_words=words.flatten(),
        )
