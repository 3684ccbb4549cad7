"""Sync-free CSR page table that produces the int32 inputs of the verify path.

State contract of batchspec/backends/base/page_table.py:8-154 and
batchspec/backends/utils/paging.py:10-277 (the caller may keep its own PageTable;
this one only removes its host round trips):
  * ``paged_kv_indptr[B+1]``, ``paged_kv_indices[sum pages]``,
    ``paged_kv_last_page_len[B]`` (int32), ``cachelens[B]``;
  * a request always holds at least one page; total tokens of request r are
    (pages_r - 1) * page_size + last_page_len[r];
  * page ids are deterministic: the k-th page of request r is r * max_pages + k;
    allocation appends at the tail, freeing pops from the tail.
The kernels never assume that id pattern (any permutation of pages works).

``DevicePageTable`` keeps that state in fixed-size device buffers and updates it
with one kernel (bsx_page_table_update): no host synchronisation per step, so the
step around it can be captured in a graph; an over-allocation is counted on the device
and raised by ``check()``.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._util import require_gpu, stream_of

_I32 = torch.int32


class DevicePageTable:
    """PageTable (batchspec/backends/base/page_table.py:8-154) without host round trips.

    Same attributes and methods as ``PageTable``; ``paged_kv_indices`` is a fixed buffer
    of max_batch_size * max_num_pages_per_request ids whose first paged_kv_indptr[-1]
    entries are the table, and ``page_manager.num_allocated_pages`` the page counts.
    ``insert_kv`` / ``delete_kv`` take an int (every request) or a per-request tensor
    and launch one kernel on the current stream.  An insert that would exceed
    max_num_pages_per_request changes nothing and is counted: ``check()`` raises the
    reference's RuntimeError for it (one host read, at a point the caller chooses)."""

    class _Pages:
        def __init__(self, counts: torch.Tensor, max_pages: int):
            self.num_allocated_pages = counts
            self.max_num_pages_per_request = max_pages

    def __init__(self, page_size: int, max_batch_size: int, max_num_pages_per_request: int,
                 device):
        self.page_size = int(page_size)
        self.max_batch_size = int(max_batch_size)
        self.max_num_pages_per_request = int(max_num_pages_per_request)
        self.device = torch.device(device)
        require_gpu("DevicePageTable", torch.empty(0, device=self.device))
        B, P = self.max_batch_size, self.max_num_pages_per_request
        self.page_manager = self._Pages(torch.empty(B, dtype=_I32, device=self.device), P)
        self.cachelens = torch.empty(B, dtype=_I32, device=self.device)
        self.paged_kv_indptr = torch.empty(B + 1, dtype=_I32, device=self.device)
        self.paged_kv_indices = torch.empty(B * P, dtype=_I32, device=self.device)
        self.paged_kv_last_page_len = torch.empty(B, dtype=_I32, device=self.device)
        self.errors = torch.zeros(1, dtype=_I32, device=self.device)
        self.clear_kv()

    def _update(self, lens, sign: int) -> None:
        if isinstance(lens, torch.Tensor) and lens.dim() > 0:
            d = lens.to(device=self.device, dtype=_I32).contiguous()
            if d.numel() != self.max_batch_size:
                raise ValueError(f"expected {self.max_batch_size} lengths, got {d.numel()}")
            dp, ds = d.data_ptr(), 0
        elif isinstance(lens, (list, tuple)):
            return self._update(torch.tensor(lens, dtype=_I32), sign)
        else:
            dp, ds = None, int(lens)
        rc = _lib.load().bsx_page_table_update(
            self.page_manager.num_allocated_pages.data_ptr(),
            self.paged_kv_last_page_len.data_ptr(), self.cachelens.data_ptr(), dp, ds, sign,
            self.max_batch_size, self.page_size, self.max_num_pages_per_request,
            self.paged_kv_indptr.data_ptr(), self.paged_kv_indices.data_ptr(),
            self.errors.data_ptr(), stream_of(self.device))
        _lib.check(rc, "insert_kv" if sign > 0 else "delete_kv")

    def insert_kv(self, dec_lens) -> None:
        self._update(dec_lens, +1)

    def delete_kv(self, del_lens) -> None:
        self._update(del_lens, -1)

    def clear_kv(self, model: Optional[torch.nn.Module] = None) -> None:
        if model is not None:
            for layer in model.layers:
                layer.attention.kv_cache.kv_cache.zero_()
        B, P = self.max_batch_size, self.max_num_pages_per_request
        self.cachelens.zero_()
        self.page_manager.num_allocated_pages.fill_(1)
        self.paged_kv_last_page_len.zero_()
        torch.arange(B + 1, dtype=_I32, device=self.device, out=self.paged_kv_indptr)
        torch.arange(0, B * P, P, dtype=_I32, device=self.device, out=self.paged_kv_indices[:B])

    def check(self) -> None:
        """Raise the reference's error if an insert was refused since the last check."""
        n = int(self.errors.item())
        if n:
            self.errors.zero_()
            raise RuntimeError("allocate_counts would exceed max_num_pages_per_request.")
