"""CSR page table that produces the int32 inputs of the verify path.

Same contract as batchspec/backends/base/page_table.py:8-154 and
batchspec/backends/utils/paging.py:10-277:
  * ``paged_kv_indptr[B+1]``, ``paged_kv_indices[sum pages]``,
    ``paged_kv_last_page_len[B]`` (int32), ``cachelens[B]``;
  * a request always holds at least one page; total tokens of request r are
    (pages_r - 1) * page_size + last_page_len[r];
  * page ids are deterministic: the k-th page of request r is r * max_pages + k;
    allocation appends at the tail, freeing pops from the tail.
The kernels never assume that id pattern (any permutation of pages works).

``DevicePageTable`` keeps the same state in fixed-size device buffers and updates it
with one kernel (bsx_page_table_update): no host synchronisation per step, so the
step around it can be captured in a graph; an over-allocation is counted on the device
and raised by ``check()``.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from . import _lib
from ._util import require_gpu, stream_of

_I32 = torch.int32


def _segment_offsets(counts: torch.Tensor) -> torch.Tensor:
    """For counts [c0, c1, ...] -> [0..c0-1, 0..c1-1, ...] (int64)."""
    counts = counts.to(torch.int64)
    total = int(counts.sum().item())
    starts = torch.cumsum(counts, 0) - counts
    return torch.arange(total, device=counts.device) - torch.repeat_interleave(starts, counts)


class PageManager:
    """Per-request append-only page allocator (batchspec/backends/utils/paging.py:10-277)."""

    def __init__(self, bsz: int, max_num_pages_per_request: int, device):
        self.bsz = int(bsz)
        self.max_num_pages_per_request = int(max_num_pages_per_request)
        self.num_allocated_pages = torch.zeros(self.bsz, dtype=_I32, device=device)

    def reset(self) -> None:
        self.num_allocated_pages.fill_(0)

    def _new_ids(self, reqs: torch.Tensor, counts: torch.Tensor, old: torch.Tensor) -> torch.Tensor:
        within = _segment_offsets(counts)
        req_rep = torch.repeat_interleave(reqs.to(torch.int64), counts.to(torch.int64))
        return req_rep * self.max_num_pages_per_request + old[req_rep].to(torch.int64) + within

    def allocate(self, add_counts: torch.Tensor, kv_page_indices: Optional[torch.Tensor] = None,
                 kv_page_indptr: Optional[torch.Tensor] = None):
        """Append add_counts[r] >= 0 pages to each request r.

        Without a table: returns the ids of the new pages.  With one: returns the
        updated (kv_page_indptr, kv_page_indices)."""
        dev = self.num_allocated_pages.device
        add = add_counts.to(device=dev, dtype=_I32).clamp_min(0)
        old = self.num_allocated_pages
        new = old + add
        if bool((new > self.max_num_pages_per_request).any()):
            raise RuntimeError("allocate_counts would exceed max_num_pages_per_request.")
        reqs = torch.nonzero(add > 0).flatten()
        if kv_page_indices is None or kv_page_indptr is None:
            ids = self._new_ids(reqs, add[reqs], old).to(_I32) if reqs.numel() else \
                torch.empty(0, dtype=_I32, device=dev)
            self.num_allocated_pages = new
            return ids
        indptr = torch.zeros(self.bsz + 1, dtype=_I32, device=dev)
        indptr[1:] = torch.cumsum(new, 0)
        total = int(indptr[-1].item())
        indices = torch.empty(total, dtype=kv_page_indices.dtype, device=dev)
        # old pages keep their order at the head of each request's slice
        n_old = kv_page_indices.numel()
        if n_old:
            req_of = torch.searchsorted(kv_page_indptr.to(torch.int64),
                                        torch.arange(n_old, device=dev), right=True) - 1
            intra = torch.arange(n_old, device=dev) - kv_page_indptr.to(torch.int64)[req_of]
            indices[indptr.to(torch.int64)[req_of] + intra] = kv_page_indices
        if reqs.numel():
            cnt = add[reqs]
            dst = torch.repeat_interleave(indptr.to(torch.int64)[reqs] + old[reqs].to(torch.int64),
                                          cnt.to(torch.int64)) + _segment_offsets(cnt)
            indices[dst] = self._new_ids(reqs, cnt, old).to(indices.dtype)
        self.num_allocated_pages = new
        return indptr, indices

    def free(self, remove_counts: torch.Tensor, kv_page_indices: torch.Tensor,
             kv_page_indptr: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Pop remove_counts[r] pages from the tail of each request r."""
        dev = self.num_allocated_pages.device
        rem = remove_counts.to(device=dev, dtype=_I32).clamp_min(0)
        old = self.num_allocated_pages
        if bool((rem > old).any()):
            raise RuntimeError("free_counts would free more pages than allocated.")
        new = old - rem
        indptr = torch.zeros(self.bsz + 1, dtype=_I32, device=dev)
        indptr[1:] = torch.cumsum(new, 0)
        n_old = kv_page_indices.numel()
        req_of = torch.searchsorted(kv_page_indptr.to(torch.int64), torch.arange(n_old, device=dev),
                                    right=True) - 1
        intra = torch.arange(n_old, device=dev) - kv_page_indptr.to(torch.int64)[req_of]
        keep = intra < new.to(torch.int64)[req_of]
        self.num_allocated_pages = new
        return indptr, kv_page_indices[keep]


class PageTable:
    """Page table state of one batch (batchspec/backends/base/page_table.py:8-154)."""

    def __init__(self, page_size: int, max_batch_size: int, max_num_pages_per_request: int,
                 device):
        self.page_size = int(page_size)
        self.max_batch_size = int(max_batch_size)
        self.max_num_pages_per_request = int(max_num_pages_per_request)
        self.device = torch.device(device)
        self.page_manager = PageManager(max_batch_size, max_num_pages_per_request, self.device)
        self.cachelens = torch.zeros(self.max_batch_size, dtype=_I32, device=self.device)
        self.page_manager.reset()
        self.paged_kv_indptr = torch.arange(self.max_batch_size + 1, dtype=_I32, device=self.device)
        self.paged_kv_indices = torch.empty(max_batch_size * max_num_pages_per_request, dtype=_I32,
                                            device=self.device)
        self.paged_kv_last_page_len = torch.empty(self.max_batch_size, dtype=_I32,
                                                  device=self.device)

    def _as_len_tensor(self, lens: Union[int, list, torch.Tensor]) -> torch.Tensor:
        if isinstance(lens, torch.Tensor):
            t = lens.to(device=self.device, dtype=_I32)
        else:
            t = torch.tensor(lens, device=self.device, dtype=_I32)
        return t.expand(self.max_batch_size) if t.dim() == 0 else t

    def _tail_state(self, total: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        ps = self.page_size
        pos = total > 0
        full = torch.where(pos, torch.div(total - 1, ps, rounding_mode="floor"),
                           torch.zeros_like(total)).to(_I32)
        tail = torch.where(pos, (total - 1) % ps + 1, torch.zeros_like(total)).to(_I32)
        return full, tail

    def insert_kv(self, dec_lens) -> None:
        """Account for dec_lens new tokens per request, allocating pages as needed."""
        dec = self._as_len_tensor(dec_lens)
        if bool((dec <= 0).all()):
            return
        old_full = self.page_manager.num_allocated_pages - 1
        total = old_full * self.page_size + self.paged_kv_last_page_len + dec
        new_full, new_tail = self._tail_state(total)
        add = (new_full - old_full).clamp_min(0).to(_I32)
        if int(add.max().item()) > 0:
            self.paged_kv_indptr, self.paged_kv_indices = self.page_manager.allocate(
                add, self.paged_kv_indices, self.paged_kv_indptr)
        self.paged_kv_last_page_len = new_tail
        self.cachelens = (self.cachelens + dec).clamp_min(0)

    def delete_kv(self, del_lens) -> None:
        """Drop del_lens tokens from the tail of each request, freeing pages."""
        dl = self._as_len_tensor(del_lens)
        if bool((dl <= 0).all()):
            return
        old_full = self.page_manager.num_allocated_pages - 1
        total = (old_full * self.page_size + self.paged_kv_last_page_len - dl).clamp_min(0)
        new_full, new_tail = self._tail_state(total)
        rem = (old_full - new_full).clamp_min(0).to(_I32)
        if int(rem.max().item()) > 0:
            self.paged_kv_indptr, self.paged_kv_indices = self.page_manager.free(
                rem, self.paged_kv_indices, self.paged_kv_indptr)
        self.paged_kv_last_page_len = new_tail
        self.cachelens = (self.cachelens - dl).clamp_min(0)

    def clear_kv(self, model: Optional[torch.nn.Module] = None) -> None:
        """Reset to one empty page per request (and zero the model's caches)."""
        if model is not None:
            for layer in model.layers:
                layer.attention.kv_cache.kv_cache.zero_()
        self.cachelens.zero_()
        self.page_manager.reset()
        self.paged_kv_indptr = torch.arange(self.max_batch_size + 1, dtype=_I32, device=self.device)
        self.paged_kv_indices = self.page_manager.allocate(
            torch.ones(self.max_batch_size, dtype=_I32, device=self.device))
        self.paged_kv_last_page_len.zero_()


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
