"""ORACLE — TEST INFRASTRUCTURE ONLY.  Paged KV append restated with numpy.

Follows StandardKVCache.update (batchspec/models/modules/kv_cache.py:47-84):
  seq_len[b]  = get_seq_lens(kv_indptr, last_page_len, page_size)  (kv_cache.py:66-70)
  (batch_indices, positions) = get_batch_indices_positions(append_indptr, seq_lens, nnz)
      token i of request b -> position seq_len[b] - n_b + (i - append_indptr[b])
  append_paged_kv_cache (NHD): cache[indices[indptr[b] + pos // ps], 0|1, pos % ps] = k|v[i]
The page table already includes the appended tokens (insert_kv runs first:
batchspec/backends/continuous/batch_builder.py:75, mtp_engine.py:419).
"""
from __future__ import annotations

import numpy as np

from .attention import seq_lens as get_seq_lens


def get_batch_indices_positions(append_indptr, seq_lens, nnz: int):
    ap = np.asarray(append_indptr, dtype=np.int64)
    sl = np.asarray(seq_lens, dtype=np.int64)
    bidx = np.zeros(nnz, dtype=np.int32)
    pos = np.zeros(nnz, dtype=np.int32)
    for b in range(ap.shape[0] - 1):
        n = ap[b + 1] - ap[b]
        for i in range(ap[b], ap[b + 1]):
            if i < nnz:
                bidx[i] = b
                pos[i] = sl[b] - n + (i - ap[b])
    return bidx, pos


def append_paged_kv_cache(k, v, batch_indices, positions, cache, kv_indices, kv_indptr,
                          page_size: int) -> np.ndarray:
    """Returns a new cache array with the rows written (input left untouched)."""
    out = np.array(cache, copy=True)
    kv_indices = np.asarray(kv_indices)
    kv_indptr = np.asarray(kv_indptr)
    for i in range(len(batch_indices)):
        b, p = int(batch_indices[i]), int(positions[i])
        page = kv_indices[kv_indptr[b] + p // page_size]
        out[page, 0, p % page_size] = k[i]
        out[page, 1, p % page_size] = v[i]
    return out


def update(k, v, append_indptr, cache, kv_indptr, kv_indices, kv_last_page_len, page_size: int):
    """StandardKVCache.update as one call."""
    nnz = int(np.asarray(append_indptr)[-1])
    sl = get_seq_lens(kv_indptr, kv_last_page_len, page_size)
    bidx, pos = get_batch_indices_positions(append_indptr, sl, nnz)
    return append_paged_kv_cache(k, v, bidx, pos, cache, kv_indices, kv_indptr, page_size)
