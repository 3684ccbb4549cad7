"""Paged KV append behind the FlashInfer functions BatchSpec imports.

batchspec/models/modules/kv_cache.py:8-12 imports ``get_batch_indices_positions``,
``get_seq_lens`` and ``append_paged_kv_cache`` from flashinfer and calls them from
``StandardKVCache.update`` (kv_cache.py:47-84).  The same three names are provided
here, plus ``StandardKVCache`` whose ``update`` runs the fused single-kernel append
(no host read of ``kv_append_indptr[-1]``, kv_cache.py:71).
"""
from __future__ import annotations

from typing import Tuple, Union

import torch

from . import _lib
from ._util import require_gpu, stream_of


def _i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    return t.contiguous()


def get_seq_lens(kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor,
                 page_size: int) -> torch.Tensor:
    """seq_lens[b] = (pages_b - 1) * page_size + last_page_len[b] (0 without pages)."""
    dev = require_gpu("get_seq_lens", kv_indptr, kv_last_page_len)
    kv_indptr = _i32(kv_indptr, "kv_indptr")
    last = _i32(kv_last_page_len, "kv_last_page_len")
    batch = kv_indptr.numel() - 1
    out = torch.empty(max(batch, 0), dtype=torch.int32, device=dev)
    rc = _lib.load().bsx_get_seq_lens(kv_indptr.data_ptr(), last.data_ptr(), batch,
                                      int(page_size), out.data_ptr(), stream_of(dev))
    _lib.check(rc, "get_seq_lens")
    return out


def get_batch_indices_positions(append_indptr: torch.Tensor, seq_lens: torch.Tensor,
                                nnz: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Request index and destination position of each of the nnz appended tokens."""
    dev = require_gpu("get_batch_indices_positions", append_indptr, seq_lens)
    append_indptr = _i32(append_indptr, "append_indptr")
    seq_lens = _i32(seq_lens, "seq_lens")
    batch = append_indptr.numel() - 1
    bidx = torch.empty(int(nnz), dtype=torch.int32, device=dev)
    pos = torch.empty(int(nnz), dtype=torch.int32, device=dev)
    rc = _lib.load().bsx_get_batch_indices_positions(append_indptr.data_ptr(), seq_lens.data_ptr(),
                                                     batch, int(nnz), bidx.data_ptr(),
                                                     pos.data_ptr(), stream_of(dev))
    _lib.check(rc, "get_batch_indices_positions")
    return bidx, pos


def _cache_views(paged_kv_cache) -> Tuple[torch.Tensor, torch.Tensor, int, int, int, int]:
    """(k view, v view, page stride, page_size, heads, head_dim) of an NHD cache."""
    if isinstance(paged_kv_cache, (tuple, list)):
        k, v = paged_kv_cache
        if k.dim() != 4 or k.shape != v.shape or k.stride() != v.stride():
            raise ValueError("k/v caches must both be [P, page_size, H, D] with equal strides")
        P, ps, H, D = k.shape
        if k.stride()[1:] != (H * D, D, 1):
            raise ValueError("k/v caches must be dense within a page")
        return k, v, k.stride(0), ps, H, D
    c = paged_kv_cache
    if c.dim() != 5 or c.shape[1] != 2:
        raise ValueError(f"paged_kv_cache must be [P, 2, page_size, H, D], got {tuple(c.shape)}")
    P, _, ps, H, D = c.shape
    if c.stride()[1:] != (ps * H * D, H * D, D, 1):
        raise ValueError("paged_kv_cache must be dense within a page")
    return c[:, 0], c[:, 1], c.stride(0), ps, H, D


def _check_kv_rows(x: torch.Tensor, H: int, D: int, name: str) -> torch.Tensor:
    if x.dim() != 3 or tuple(x.shape[1:]) != (H, D):
        raise ValueError(f"{name} must be [nnz, {H}, {D}], got {tuple(x.shape)}")
    if x.stride(2) != 1 or x.stride(1) != D:
        x = x.contiguous()
    return x


def append_paged_kv_cache(append_key: torch.Tensor, append_value: torch.Tensor,
                          batch_indices: torch.Tensor, positions: torch.Tensor,
                          paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
                          kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
                          kv_last_page_len: torch.Tensor, kv_layout: str = "NHD") -> None:
    """Scatter append_key/append_value rows into their (page, slot) of the cache."""
    if kv_layout != "NHD":
        raise NotImplementedError("only the NHD layout is implemented")
    k_c, v_c, page_stride, ps, H, D = _cache_views(paged_kv_cache)
    dev = require_gpu("append_paged_kv_cache", append_key, append_value, batch_indices, positions,
                      k_c, kv_indices, kv_indptr, kv_last_page_len)
    if append_key.dtype != k_c.dtype or append_value.dtype != k_c.dtype:
        raise ValueError("append_key/append_value must have the cache dtype")
    k = _check_kv_rows(append_key, H, D, "append_key")
    v = _check_kv_rows(append_value, H, D, "append_value")
    nnz = k.shape[0]
    if v.shape[0] != nnz or batch_indices.numel() < nnz or positions.numel() < nnz:
        raise ValueError("append_key, append_value, batch_indices and positions disagree on nnz")
    rc = _lib.load().bsx_append_paged_kv_cache(
        k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0),
        _i32(batch_indices, "batch_indices").data_ptr(), _i32(positions, "positions").data_ptr(),
        nnz, k_c.data_ptr(), v_c.data_ptr(), page_stride, _i32(kv_indices, "kv_indices").data_ptr(),
        _i32(kv_indptr, "kv_indptr").data_ptr(), H, D, ps, k.element_size(), stream_of(dev))
    _lib.check(rc, "append_paged_kv_cache")


def append_kv(k: torch.Tensor, v: torch.Tensor, kv_append_indptr: torch.Tensor,
              paged_kv_cache, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
              kv_last_page_len: torch.Tensor) -> None:
    """Fused append: positions derived on device from the page table (one kernel)."""
    k_c, v_c, page_stride, ps, H, D = _cache_views(paged_kv_cache)
    dev = require_gpu("append_kv", k, v, kv_append_indptr, k_c, kv_indptr, kv_indices,
                      kv_last_page_len)
    if k.dtype != k_c.dtype or v.dtype != k_c.dtype:
        raise ValueError("k/v must have the cache dtype")
    k = _check_kv_rows(k, H, D, "k")
    v = _check_kv_rows(v, H, D, "v")
    if k.shape[0] != v.shape[0]:
        raise ValueError("k and v disagree on nnz")
    batch = kv_append_indptr.numel() - 1
    rc = _lib.load().bsx_kv_append(
        k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0),
        _i32(kv_append_indptr, "kv_append_indptr").data_ptr(),
        _i32(kv_indptr, "kv_indptr").data_ptr(), _i32(kv_indices, "kv_indices").data_ptr(),
        _i32(kv_last_page_len, "kv_last_page_len").data_ptr(), batch, k.shape[0],
        k_c.data_ptr(), v_c.data_ptr(), page_stride, H, D, ps, k.element_size(), stream_of(dev))
    _lib.check(rc, "append_kv")


class StandardKVCache(torch.nn.Module):
    """Paged KV storage [max_num_pages, 2, page_size, n_heads, head_dim]
    (batchspec/models/modules/kv_cache.py:18-45) with a fused ``update``."""

    def __init__(self, max_num_pages: int, page_size: int, n_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device=None):
        super().__init__()
        shape = (max_num_pages, 2, page_size, n_heads, head_dim)
        self.register_buffer("kv_cache", torch.empty(shape, dtype=dtype, device=device))
        self.page_size = page_size

    def update(self, k: torch.Tensor, v: torch.Tensor, kv_append_indptr: torch.Tensor,
               kv_page_table) -> torch.Tensor:
        """Append k/v [nnz, H, D] at the tail of each request; returns the cache."""
        append_kv(k, v, kv_append_indptr, self.kv_cache, kv_page_table.paged_kv_indptr,
                  kv_page_table.paged_kv_indices, kv_page_table.paged_kv_last_page_len)
        return self.kv_cache
