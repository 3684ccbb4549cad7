"""Producers of the verify-step attention masks and position ids.

* ``mtp_attn_mask_and_position_ids`` — the (k+1)^2 interleaved MTP pattern of
  batchspec/backends/mtp_engine.py:172-208: row i (group g_i = i // (k+1), slot
  r_i = i % (k+1)) sees column j iff (r_j == 0 and j <= i) or
  (g_i == g_j and 1 <= r_j <= r_i); position_ids[i] = g_i + r_i.
* ``mtp_verify_custom_mask`` — the flattened per-request mask
  cat(ones(S, cachelen_b), common_mask) of mtp_engine.py:410-417.
* ``interleave_mask_tokens`` — mtp_engine.py:210-247.
* ``tree_mask_words`` — ancestor-or-self bit words of a draft tree given by a parent
  array (EAGLE-style verification), one uint32 per node, bit j = node j.
The bit words are what ``BatchPrefillWithPagedKVCacheWrapper.plan(tree_mask_words=...)``
consumes; they replace the O(qo * kv) bool mask.
"""
from __future__ import annotations

from typing import Sequence, Tuple

import numpy as np
import torch


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


def interleave_mask_tokens(input_ids: torch.Tensor, draft_length: int, mask_token_id: int,
                           dtype: torch.dtype = torch.bfloat16) -> Tuple[torch.Tensor, torch.Tensor]:
    B, L = input_ids.shape
    D = draft_length
    out = torch.full((B, L * (D + 1)), mask_token_id, dtype=input_ids.dtype, device=input_ids.device)
    out.view(B, L, D + 1)[:, :, 0] = input_ids
    gate = torch.ones((B, L * (D + 1)), dtype=dtype, device=input_ids.device)
    gate.view(B, L, D + 1)[:, :, 0] = 0
    return out, gate[..., None]


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
