"""ORACLE — TEST INFRASTRUCTURE ONLY.  Acceptance restated on the CPU.

* ``greedy_posterior`` — batchspec/backends/mtp_engine.py:553-560 (greedy branch) with
  the argmax of mtp_engine.py:747 (torch.argmax semantics: first maximum, NaN is the
  maximum) — numpy.
* ``chain_probs`` / ``chain_logits`` / ``softmax`` / ``tree_draw`` / ``exp2`` — the
  canonical stochastic acceptance of accept.c (ctypes), which restates
  mtp_engine.py:561-575 and batchspec/backends/utils/sampling.py:18-58.
* ``filter_row`` / ``filtered_probs`` / ``chain_filtered`` / ``sample`` / ``fx_draw`` —
  the top-k / top-p renormalisation (sampling.py:50-56), non-greedy sample()
  (sampling.py:61-115) and the acceptance fed filtered distributions, from filter.c.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import numpy as np

_SO = Path(__file__).resolve().parent / "liboracle.so"
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _SO.exists():
            from .build import build
            build()
        L = ctypes.CDLL(str(_SO))
        L.oc_exp2.restype = c_float
        L.oc_exp2.argtypes = [c_float]
        L.oc_softmax.argtypes = [c_void_p, c_int64, c_int64, c_float, c_void_p]
        L.oc_row_stats.argtypes = [c_void_p, c_int64, c_float, c_void_p, c_void_p]
        L.oc_tree_draw.restype = c_int64
        L.oc_tree_draw.argtypes = [c_void_p, c_int64, c_float]
        L.oc_chain_probs.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int64,
                                     c_void_p, c_void_p, c_void_p]
        L.oc_chain_logits.argtypes = [c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_int, c_int,
                                      c_int64, c_void_p, c_void_p, c_void_p]
        L.oc_okey.restype = ctypes.c_uint32
        L.oc_okey.argtypes = [c_float]
        L.oc_u64_to_f32.restype = c_float
        L.oc_u64_to_f32.argtypes = [ctypes.c_uint64]
        L.oc_filter_row.argtypes = [c_void_p, c_int64, c_float, c_int, c_float, c_void_p, c_void_p,
                                    c_void_p, c_void_p]
        L.oc_fx_draw.restype = c_int64
        L.oc_fx_draw.argtypes = [c_void_p, c_int64, c_float]
        L.oc_filtered_probs.argtypes = [c_void_p, c_int64, c_int64, c_float, c_int, c_float, c_void_p]
        L.oc_chain_filtered.argtypes = [c_void_p, c_void_p, c_void_p, c_float, c_int, c_float,
                                        c_void_p, c_int, c_int, c_int64, c_void_p, c_void_p,
                                        c_void_p]
        L.oc_sample.argtypes = [c_void_p, c_int64, c_int64, c_float, c_int, c_float, c_void_p,
                                c_void_p]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def exp2(y: float) -> float:
    return float(lib().oc_exp2(float(np.float32(y))))


def exp2_array(y: np.ndarray) -> np.ndarray:
    f = lib().oc_exp2
    return np.array([f(float(v)) for v in np.asarray(y, dtype=np.float32).ravel()],
                    dtype=np.float32).reshape(np.shape(y))


def softmax(logits: np.ndarray, temperature: float = 1.0) -> np.ndarray:
    x = _f32(logits)
    V = x.shape[-1]
    out = np.empty_like(x)
    lib().oc_softmax(x.ctypes.data, x.size // V, V, float(temperature), out.ctypes.data)
    return out


def row_stats(row: np.ndarray, temperature: float = 1.0):
    x = _f32(row)
    c = np.float32(np.float32(float.fromhex("0x1.715476p+0"))
                   * (np.float32(1.0) / np.float32(temperature)))
    m = np.zeros(1, np.float32)
    z = np.zeros(1, np.float32)
    lib().oc_row_stats(x.ctypes.data, x.size, float(c), m.ctypes.data, z.ctypes.data)
    return float(m[0]), float(z[0])


def tree_draw(weights: np.ndarray, u: float) -> int:
    w = _f32(weights)
    return int(lib().oc_tree_draw(w.ctypes.data, w.size, float(np.float32(u))))


def chain_probs(draft_probs, draft_ids, target_probs, uniforms):
    """-> (out_ids [B,k+1] int32, accepted [B] int32, emitted [B] int32)"""
    ids = np.ascontiguousarray(np.asarray(draft_ids, dtype=np.int64))
    B, k = ids.shape
    tp = _f32(target_probs)
    V = tp.shape[-1]
    dp = None if draft_probs is None else _f32(draft_probs)
    u = _f32(uniforms)
    out = np.empty((B, k + 1), np.int32)
    acc = np.empty(B, np.int32)
    emi = np.empty(B, np.int32)
    lib().oc_chain_probs(None if dp is None else dp.ctypes.data, ids.ctypes.data, tp.ctypes.data,
                         u.ctypes.data, B, k, V, out.ctypes.data, acc.ctypes.data, emi.ctypes.data)
    return out, acc, emi


def chain_logits(draft_logits, draft_ids, target_logits, temperature, uniforms):
    """Logits (any float dtype, widened exactly to fp32) -> chain_probs of their softmax."""
    ids = np.ascontiguousarray(np.asarray(draft_ids, dtype=np.int64))
    B, k = ids.shape
    tl = _f32(target_logits)
    V = tl.shape[-1]
    dl = None if draft_logits is None else _f32(draft_logits)
    u = _f32(uniforms)
    out = np.empty((B, k + 1), np.int32)
    acc = np.empty(B, np.int32)
    emi = np.empty(B, np.int32)
    lib().oc_chain_logits(None if dl is None else dl.ctypes.data, ids.ctypes.data, tl.ctypes.data,
                          float(temperature), u.ctypes.data, B, k, V, out.ctypes.data,
                          acc.ctypes.data, emi.ctypes.data)
    return out, acc, emi


def argmax(logits: np.ndarray) -> np.ndarray:
    """torch.argmax(-1): first maximum, NaN counts as the maximum (first NaN)."""
    x = np.asarray(logits, dtype=np.float32)
    return np.argmax(x, axis=-1).astype(np.int64)


def greedy_posterior(draft_tokens, target_preds, eos_token_id: int, rule: str = "reference"):
    """mtp_engine.py:553-560.  target_preds: ids [B, k+1] or logits [B, k+1, V].
    -> (bonus [B,1] int64, accept_nums [B] int64, eos_accepted [B,1] bool)"""
    draft = np.asarray(draft_tokens, dtype=np.int64)
    preds = np.asarray(target_preds)
    if preds.ndim == 3:
        preds = argmax(preds)
    preds = preds.astype(np.int64)
    B, k = draft.shape
    flags = preds[:, :k] == draft
    if rule == "reference":
        counted = flags
    else:
        counted = np.cumprod(flags, axis=1).astype(bool)
    accept = counted.sum(axis=1) + 1
    bonus = preds[np.arange(B), accept - 1]
    eos = ((draft == eos_token_id) & counted).any(axis=1)
    return bonus[:, None], accept.astype(np.int64), eos[:, None]


def okey(x: float) -> int:
    return int(lib().oc_okey(float(np.float32(x))))


def u64_to_f32(v: int) -> float:
    return float(lib().oc_u64_to_f32(int(v)))


def filter_row(row, temperature: float, top_k: int, top_p: float):
    """-> (M, inv_k, t_key, zk_fx) of one row (the filtered distribution's parameters)."""
    x = _f32(row)
    M = np.zeros(1, np.float32)
    inv = np.zeros(1, np.float32)
    t = np.zeros(1, np.uint32)
    zk = np.zeros(1, np.uint64)
    lib().oc_filter_row(x.ctypes.data, x.size, float(temperature), int(top_k), float(top_p),
                        M.ctypes.data, inv.ctypes.data, t.ctypes.data, zk.ctypes.data)
    return float(M[0]), float(inv[0]), int(t[0]), int(zk[0])


def fx_draw(weights, u: float) -> int:
    w = _f32(weights)
    return int(lib().oc_fx_draw(w.ctypes.data, w.size, float(np.float32(u))))


def filtered_probs(logits, temperature: float, top_k: int, top_p: float) -> np.ndarray:
    x = _f32(logits)
    V = x.shape[-1]
    out = np.empty_like(x)
    lib().oc_filtered_probs(x.ctypes.data, x.size // V, V, float(temperature), int(top_k),
                            float(top_p), out.ctypes.data)
    return out


def chain_filtered(draft_logits, draft_ids, target_logits, temperature, top_k, top_p, uniforms):
    """Chain acceptance over top-k / top-p filtered softmax distributions."""
    ids = np.ascontiguousarray(np.asarray(draft_ids, dtype=np.int64))
    B, k = ids.shape
    tl = _f32(target_logits)
    V = tl.shape[-1]
    dl = None if draft_logits is None else _f32(draft_logits)
    u = _f32(uniforms)
    out = np.empty((B, k + 1), np.int32)
    acc = np.empty(B, np.int32)
    emi = np.empty(B, np.int32)
    lib().oc_chain_filtered(None if dl is None else dl.ctypes.data, ids.ctypes.data,
                            tl.ctypes.data, float(temperature), int(top_k), float(top_p),
                            u.ctypes.data, B, k, V, out.ctypes.data, acc.ctypes.data,
                            emi.ctypes.data)
    return out, acc, emi


def sample(logits, temperature: float, top_k: int, top_p: float, uniforms) -> np.ndarray:
    """sample() for temperature > 0: one draw per row of [rows, V] with uniforms[rows]."""
    x = _f32(logits)
    V = x.shape[-1]
    rows = x.size // V
    u = _f32(uniforms).reshape(-1)
    if u.size != rows:
        raise ValueError("one uniform per row")
    out = np.empty(rows, np.int64)
    lib().oc_sample(x.ctypes.data, rows, V, float(temperature), int(top_k), float(top_p),
                    u.ctypes.data, out.ctypes.data)
    return out
