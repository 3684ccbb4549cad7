"""ORACLE — TEST INFRASTRUCTURE ONLY.  CSR page table restated with plain numpy loops.

Follows batchspec/backends/utils/paging.py:10-277 (PageManager: page k of request r
has id r * max_pages + k; allocate appends at the tail and raises past max_pages,
free pops from the tail and raises when freeing more than held) and
batchspec/backends/base/page_table.py:55-154 (insert_kv / delete_kv / clear_kv:
total = (pages - 1) * page_size + last_page_len, at least one page per request).
"""
from __future__ import annotations

import numpy as np


class Pages:
    def __init__(self, bsz: int, max_pages: int, page_size: int):
        self.bsz, self.max_pages, self.page_size = bsz, max_pages, page_size
        self.pages = [[] for _ in range(bsz)]  # page ids per request, in order
        self.last = [0] * bsz

    # paging.py:155-237
    def allocate(self, add_counts):
        new_ids = []
        for r, a in enumerate(add_counts):
            a = max(int(a), 0)
            if len(self.pages[r]) + a > self.max_pages:
                raise RuntimeError("allocate_counts would exceed max_num_pages_per_request.")
        for r, a in enumerate(add_counts):
            for _ in range(max(int(a), 0)):
                pid = r * self.max_pages + len(self.pages[r])
                self.pages[r].append(pid)
                new_ids.append(pid)
        return new_ids

    # paging.py:239-277
    def free(self, remove_counts):
        for r, a in enumerate(remove_counts):
            if max(int(a), 0) > len(self.pages[r]):
                raise RuntimeError("free_counts would free more pages than allocated.")
        for r, a in enumerate(remove_counts):
            for _ in range(max(int(a), 0)):
                self.pages[r].pop()

    def table(self):
        counts = [len(p) for p in self.pages]
        indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        indices = np.array([pid for p in self.pages for pid in p], dtype=np.int32)
        return indptr, indices, np.array(self.last, dtype=np.int32)

    def total(self, r: int) -> int:
        return (len(self.pages[r]) - 1) * self.page_size + self.last[r]

    def _retarget(self, r: int, total: int):
        total = max(total, 0)
        full = (total - 1) // self.page_size if total > 0 else 0
        tail = (total - 1) % self.page_size + 1 if total > 0 else 0
        return full, tail

    # page_table.py:55-94
    def insert_kv(self, dec):
        dec = [int(d) for d in dec]
        if all(d <= 0 for d in dec):
            return
        add = []
        tails = []
        for r in range(self.bsz):
            full, tail = self._retarget(r, self.total(r) + dec[r])
            add.append(max(full - (len(self.pages[r]) - 1), 0))
            tails.append(tail)
        self.allocate(add)
        self.last = tails

    # page_table.py:96-137
    def delete_kv(self, dels):
        dels = [int(d) for d in dels]
        if all(d <= 0 for d in dels):
            return
        rem = []
        tails = []
        for r in range(self.bsz):
            full, tail = self._retarget(r, self.total(r) - dels[r])
            rem.append(max((len(self.pages[r]) - 1) - full, 0))
            tails.append(tail)
        self.free(rem)
        self.last = tails

    # page_table.py:139-154
    def clear_kv(self):
        self.pages = [[r * self.max_pages] for r in range(self.bsz)]
        self.last = [0] * self.bsz
