"""ORACLE — TEST INFRASTRUCTURE ONLY.  fp32 eager paged-gather attention.

Restates what BatchSpec asks of FlashInfer's BatchPrefillWithPagedKVCacheWrapper:
  * plan arguments: batchspec/backends/standard_engine.py:132-143 (causal=True) and
    batchspec/backends/mtp_engine.py:420-432 (custom_mask = cat(ones(qo, cachelen),
    common_mask) per request, flattened, mtp_engine.py:410-417);
  * run: batchspec/models/modules/attention/standard.py:69 — q [nnz, Hq, D],
    cache [P, 2, page_size, Hkv, D] (NHD, batchspec/models/modules/kv_cache.py:43);
  * kv length per request = (pages - 1) * page_size + last_page_len
    (get_seq_lens, kv_cache.py:66-70), token j of request b lives in page
    kv_indices[kv_indptr[b] + j // page_size], slot j % page_size;
  * causal masks are aligned bottom-right: query t sees j <= kv_len - qo_len + t;
  * GQA: query head h reads kv head h // (Hq / Hkv); default scale 1/sqrt(D).
The sink + window view keeps tokens j < sink or j >= kv_len - window (MagicDec-style
StreamingLLM draft KV, batchspec/models/modules/kv_cache.py:87-295, read as a view
over the same page table instead of a compaction), causal over the last qo_len.
"""
from __future__ import annotations

from typing import Optional

import numpy as np


def seq_lens(kv_indptr: np.ndarray, kv_last_page_len: np.ndarray, page_size: int) -> np.ndarray:
    np_ = np.diff(np.asarray(kv_indptr, dtype=np.int64))
    last = np.asarray(kv_last_page_len, dtype=np.int64)[: np_.shape[0]]
    return np.where(np_ > 0, (np_ - 1) * page_size + last, 0)


def token_slots(kv_indptr, kv_indices, page_size: int, b: int, kv_len: int):
    """(page id, slot) of tokens 0..kv_len-1 of request b."""
    j = np.arange(kv_len)
    pages = np.asarray(kv_indices)[int(kv_indptr[b]) + j // page_size]
    return pages, j % page_size


def gather_kv(cache: np.ndarray, kv_indptr, kv_indices, page_size: int, b: int, kv_len: int):
    pages, slots = token_slots(kv_indptr, kv_indices, page_size, b, kv_len)
    return cache[pages, 0, slots], cache[pages, 1, slots]  # [L, Hkv, D] each


def visibility(mode: str, qo_len: int, kv_len: int, custom: Optional[np.ndarray] = None,
               sink: int = 0, window: int = 0) -> np.ndarray:
    """Bool [qo_len, kv_len]: may query t attend to kv token j."""
    t = np.arange(qo_len)[:, None]
    j = np.arange(kv_len)[None, :]
    diag = kv_len - qo_len
    if mode == "none":
        return np.ones((qo_len, kv_len), dtype=bool)
    if mode == "causal":
        return j <= diag + t
    if mode == "custom":
        return np.asarray(custom, dtype=bool).reshape(qo_len, kv_len)
    if mode == "streaming":
        return ((j < sink) | (j >= kv_len - window)) & (j <= diag + t)
    raise ValueError(mode)


def verify_attention(q: np.ndarray, cache: np.ndarray, qo_indptr, kv_indptr, kv_indices,
                     kv_last_page_len, page_size: int, mode: str = "causal",
                     custom_mask: Optional[np.ndarray] = None, sink: int = 0, window: int = 0,
                     sm_scale: Optional[float] = None, return_lse: bool = False):
    """out [nnz, Hq, D] fp32 (and natural-log lse [nnz, Hq]).  Rows that see no token
    output zeros (lse -inf)."""
    q = np.asarray(q, dtype=np.float32)
    cache = np.asarray(cache, dtype=np.float32)
    nnz, Hq, D = q.shape
    Hkv = cache.shape[3]
    g = Hq // Hkv
    scale = np.float32(1.0 / np.sqrt(D) if sm_scale is None else sm_scale)
    qo_indptr = np.asarray(qo_indptr, dtype=np.int64)
    lens = seq_lens(kv_indptr, kv_last_page_len, page_size)
    out = np.zeros((nnz, Hq, D), dtype=np.float32)
    lse = np.full((nnz, Hq), -np.inf, dtype=np.float32)
    moff = 0
    for b in range(qo_indptr.shape[0] - 1):
        q0, q1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        qo_len, kv_len = q1 - q0, int(lens[b])
        cm = None
        if mode == "custom":
            cm = custom_mask[moff: moff + qo_len * kv_len]
            moff += qo_len * kv_len
        if qo_len == 0 or kv_len == 0:
            continue
        K, Vv = gather_kv(cache, kv_indptr, kv_indices, page_size, b, kv_len)
        vis = visibility(mode, qo_len, kv_len, cm, sink, window)
        for h in range(Hq):
            kh = h // g
            s = (q[q0:q1, h, :] @ K[:, kh, :].T) * scale  # [qo, L]
            s = np.where(vis, s, -np.inf).astype(np.float32)
            m = s.max(axis=1, keepdims=True)
            has = np.isfinite(m[:, 0])
            m = np.where(np.isfinite(m), m, 0.0).astype(np.float32)
            p = np.exp(s - m).astype(np.float32)
            l = p.sum(axis=1, keepdims=True)
            o = (p @ Vv[:, kh, :]) / np.where(l > 0, l, 1.0)
            out[q0:q1, h, :] = np.where(has[:, None], o, 0.0)
            lse[q0:q1, h] = np.where(has, (m[:, 0] + np.log(np.where(l[:, 0] > 0, l[:, 0], 1.0))),
                                     -np.inf)
    return (out, lse) if return_lse else out
