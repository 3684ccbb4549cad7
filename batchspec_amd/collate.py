"""Accepted-KV compaction after a verify step.

Replaces MTPEngine.collate_accepted_kv_cache (batchspec/backends/mtp_engine.py:577-631):
the KV rows of each request's accepted regular tokens (positions
prev + i*(draft_length+1), i < accept_nums[b]) move to positions prev + i in every
layer's cache, in one launch, in place, through the page table; then the page table
drops the rest of the (k+1)^2 inserted rows (delete_kv, mtp_engine.py:630-631).
"""
from __future__ import annotations

from typing import Sequence, Union

import torch

from . import _lib
from ._util import require_gpu, stream_of

_BASES: dict = {}


def _layer_views(kv_caches: Union[torch.Tensor, Sequence[torch.Tensor]]):
    """Per-layer [P, 2, ps, H, D] caches -> (k bases, v bases, page stride, ps, H, D, elem)."""
    caches = [kv_caches] if isinstance(kv_caches, torch.Tensor) and kv_caches.dim() == 5 \
        else list(kv_caches)
    if not caches:
        raise ValueError("no kv caches")
    c0 = caches[0]
    if c0.dim() != 5 or c0.shape[1] != 2:
        raise ValueError(f"kv caches must be [P, 2, page_size, H, D], got {tuple(c0.shape)}")
    P, _, ps, H, D = c0.shape
    for c in caches:
        if c.shape != c0.shape or c.dtype != c0.dtype or c.stride() != c0.stride():
            raise ValueError("every layer's kv cache must share shape, dtype and strides")
        if c.stride()[1:] != (ps * H * D, H * D, D, 1):
            raise ValueError("kv cache must be dense within a page")
        if c.data_ptr() % 16:
            raise ValueError("kv cache must be 16-byte aligned")
    return caches, c0.stride(0), ps, H, D, c0.element_size()


def collate_accepted_kv_cache(accept_nums: torch.Tensor, prev_cachelens: torch.Tensor,
                              draft_length: int, kv_caches, paged_kv_indptr: torch.Tensor,
                              paged_kv_indices: torch.Tensor) -> None:
    """Move the accepted KV rows of every layer in place (see module docstring).

    kv_caches: one [P, 2, page_size, H_kv, D] tensor or a sequence of them (one per
    layer).  accept_nums [B] (any integer dtype), prev_cachelens [B] int32."""
    caches, page_stride, ps, H, D, esz = _layer_views(kv_caches)
    dev = require_gpu("collate_accepted_kv_cache", accept_nums, prev_cachelens, paged_kv_indptr,
                      paged_kv_indices, *caches)
    if accept_nums.dim() != 1 or prev_cachelens.dim() != 1 or \
            accept_nums.shape != prev_cachelens.shape:
        raise ValueError("accept_nums and prev_cachelens must be 1-D tensors of equal length")
    B = accept_nums.numel()
    if paged_kv_indptr.numel() < B + 1:
        raise ValueError("paged_kv_indptr must hold batch + 1 entries")
    acc = accept_nums.to(torch.int64).contiguous()
    prev = prev_cachelens.to(torch.int32).contiguous()
    indptr = paged_kv_indptr.to(torch.int32).contiguous()
    indices = paged_kv_indices.to(torch.int32).contiguous()
    key = (dev, tuple(c.data_ptr() for c in caches), ps, H, D, esz)
    bases = _BASES.get(key)
    if bases is None:
        vofs = ps * H * D * esz
        bases = torch.tensor([[c.data_ptr() for c in caches], [c.data_ptr() + vofs for c in caches]],
                             dtype=torch.int64, device=dev)
        _BASES.clear()
        _BASES[key] = bases
    rc = _lib.load().bsx_collate_accepted_kv(acc.data_ptr(), prev.data_ptr(), B, int(draft_length),
                                             indptr.data_ptr(), indices.data_ptr(),
                                             bases[0].data_ptr(), bases[1].data_ptr(), len(caches),
                                             page_stride, H, D, ps, esz, stream_of(dev))
    _lib.check(rc, "collate_accepted_kv_cache")


class CollateMixin:
    """Engine mixin with the reference method's signature
    (batchspec/backends/mtp_engine.py:577-631): expects ``self.draft_length``,
    ``self.model.layers[*].attention.kv_cache.kv_cache``, ``self.kv_page_table``
    (``paged_kv_indptr`` / ``paged_kv_indices``) and ``self.delete_kv``."""

    def collate_accepted_kv_cache(self, accept_nums: torch.Tensor, prev_cachelens: torch.Tensor):
        caches = [layer.attention.kv_cache.kv_cache for layer in self.model.layers]
        pt = self.kv_page_table
        collate_accepted_kv_cache(accept_nums, prev_cachelens, self.draft_length, caches,
                                  pt.paged_kv_indptr, pt.paged_kv_indices)
        inserted_len = (self.draft_length + 1) ** 2
        self.delete_kv(inserted_len - accept_nums)
