"""ORACLE — TEST INFRASTRUCTURE ONLY.  Accepted-KV compaction restated with numpy loops.

Follows MTPEngine.collate_accepted_kv_cache (batchspec/backends/mtp_engine.py:577-631):
src = prev + i*(k+1), dst = prev + i for i < accept_nums[b] (mtp_engine.py:610-618),
kv[b, dst] = kv[b, src] with the right-hand side gathered first (:626), for every
layer.  The reference addresses request b's positions in a contiguous page range
(its reshape at :624 relies on page ids r*max_pages + k); here position p of request
b is page kv_indices[kv_indptr[b] + p // page_size], slot p % page_size, which is
the same slot under that layout.
"""
from __future__ import annotations

import numpy as np


def save_indices(accept_nums, prev_cachelens, draft_length: int):
    """The source positions kept per request (the docstring's "save indices")."""
    stride = draft_length + 1
    return [[int(p) + i * stride for i in range(int(a))]
            for a, p in zip(accept_nums, prev_cachelens)]


def collate(cache, accept_nums, prev_cachelens, draft_length: int, kv_indptr, kv_indices,
            page_size: int):
    """cache [P, 2, ps, H, D] (one layer); returns a new array."""
    out = np.array(cache, copy=True)
    src_all = save_indices(accept_nums, prev_cachelens, draft_length)
    for b, srcs in enumerate(src_all):
        prev = int(prev_cachelens[b])
        rows = []
        for s in srcs:  # gather every source row first, then write
            pg = int(kv_indices[int(kv_indptr[b]) + s // page_size])
            rows.append(np.array(cache[pg, :, s % page_size]))
        for i, row in enumerate(rows):
            d = prev + i
            pg = int(kv_indices[int(kv_indptr[b]) + d // page_size])
            out[pg, :, d % page_size] = row
    return out
