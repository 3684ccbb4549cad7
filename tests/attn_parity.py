"""Discriminating parity checks of verify attention at the benchmark sizes.

Plain N(0,1)*0.5 inputs over thousands of kv tokens give a near-uniform softmax whose
output (|O| ~ 0.01) sits under the north star's 2e-2 absolute floor, so a check on
them alone cannot see a dropped mask or a lost tile.  This module supplies:

* ``plant_keys``: rewrites a batch's Q and K so that every query row has one planted
  key whose score is ln(kv_len) + 1 above the bulk (about 73% of the row's weight).
  The rows of a kv head take turns between four roles:
    0. the row's own draft token (or, for trees, an ancestor node): visible, in the
       request's last tile, so a dropped last tile or a wrong draft-block mask is O(1);
    1. a token the mask hides (the next draft token, a non-ancestor tree node, a token
       between the sink and the window): seen only when the mask is wrong;
    2. the first or last token of a segment of the plan (split-KV boundaries);
    3. a tile boundary (the last token of a 32-token tile or the first of the next).
  For the sink + window view the roles are the own token, the last hidden token
  before the window, the window's first token and the sink's last token, so an
  off-by-one at either edge of the view is O(1) too.
  Planted key directions are orthonormal per (request, kv head), and a row's query is
  its noise with the direction projected out plus beta times the direction, so the
  planted score is exact up to bf16 rounding.
* ``oracle_per_request``: the fp32 oracle run request by request on pages gathered on
  the device (config 3b's 6.4 GB cache never goes to the host whole), with optional
  mask mutations (``"nomask"`` drops the mask, ``"droplast"`` hides each request's
  last kv tile) computed from the same gathered pages, for the guards.
* ``check``: the north-star elementwise bound |gpu - ref| <= 2e-2 + 2e-2 |ref| plus
  the normalised ones max |gpu - ref| <= 2e-2 max |ref| and relative L2 <= 1e-2, and
  (when given) |lse_gpu - lse_ref| <= 5e-3 with matching -inf rows.
"""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import attention as OA

ATOL = RTOL = 2e-2
NORM_MAX = 2e-2
NORM_L2 = 1e-2
LSE_ATOL = 5e-3
TILE = 32


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def mismatch(got, ref, lse_got=None, lse_ref=None):
    """Reason the check fails, or None when it passes."""
    g = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float32)
    if not np.isfinite(g).all():
        return "non-finite output"
    err = np.abs(g - ref)
    ex = (err - (ATOL + RTOL * np.abs(ref))).max()
    if ex > 0:
        return f"elementwise bound exceeded by {ex:.4g} (max abs err {err.max():.4g})"
    scale = float(np.abs(ref).max())
    if err.max() > NORM_MAX * scale:
        return f"max err {err.max():.4g} > {NORM_MAX} * max|ref| ({scale:.4g})"
    l2 = float(np.sqrt((err.astype(np.float64) ** 2).sum() / max((ref.astype(np.float64) ** 2).sum(), 1e-30)))
    if l2 > NORM_L2:
        return f"relative L2 err {l2:.4g} > {NORM_L2}"
    if lse_ref is not None:
        lg = lse_got.float().cpu().numpy() if isinstance(lse_got, torch.Tensor) else np.asarray(lse_got)
        fin = np.isfinite(lse_ref)
        if not np.array_equal(np.isfinite(lg), fin):
            return "lse -inf rows differ"
        if fin.any():
            d = np.abs(lg[fin] - lse_ref[fin]).max()
            if d > LSE_ATOL:
                return f"lse err {d:.4g} > {LSE_ATOL}"
    return None


def check(got, ref, lse_got=None, lse_ref=None):
    why = mismatch(got, ref, lse_got, lse_ref)
    assert why is None, why
    err = np.abs(got.float().cpu().numpy() - ref)
    return float(err.max()), float(np.abs(ref).max())


def assert_discriminates(ref, mutants):
    """Each (name, mutant output[, mutant lse]) must fail the check against ref."""
    ref_o, ref_l = ref
    for name, mo, ml in mutants:
        why = mismatch(mo, ref_o, ml, ref_l)
        assert why is not None, f"the check cannot tell '{name}' from the reference"
        say(f"  guard '{name}': rejected ({why})")


def _tree_words(b, r):
    q0, q1 = int(b.qo_indptr[r]), int(b.qo_indptr[r + 1])
    return np.asarray(b.mask_words[q0:q1], dtype=np.uint64)


def segment_boundaries(plan_blob, plan, r, kv_len, segments=None):
    """First and last kv token of each segment of request r, from a host plan's blob or
    from a segment list [S, 4] = (request, first tile, end tile, slot)."""
    if segments is not None:
        segs = np.asarray(segments).reshape(-1, 4)
    elif plan_blob is None:
        return []
    else:
        segs = plan_blob[plan.off_segments: plan.off_segments + 4 * plan.num_segments].reshape(-1, 4)
    out = []
    for b, t0, t1, _ in segs:
        if b != r or t1 <= t0:
            continue
        out.append(int(t0) * TILE)
        out.append(min(int(t1) * TILE, kv_len) - 1)
    return sorted(set(out))


def plant_keys(b, mode="causal", plan_blob=None, plan=None, seed=0, sink=0, window=0,
               beta=4.0, margin=1.0, segments=None):
    """Rewrite b.q and b.cache (device tensors) in place; returns the planted targets
    {(request, kv head, row): position} for diagnostics.  Segment boundaries come from
    a host plan (plan_blob, plan) or a segment list (segments, e.g. a device plan's)."""
    rng = np.random.default_rng(seed)
    dev = b.q.device
    Hq, Hkv, D, ps = b.num_qo_heads, b.num_kv_heads, b.head_dim, b.page_size
    g = Hq // Hkv
    qo = b.qo_indptr.cpu().numpy().astype(np.int64)
    kvp = b.kv_indptr.cpu().numpy().astype(np.int64)
    idx = b.kv_indices.cpu().numpy().astype(np.int64)
    lens = b.kv_lens
    sm = 1.0 / np.sqrt(D)
    q_rows, q_heads, q_vals = [], [], []
    k_pages, k_slots, k_heads, k_vals = [], [], [], []
    targets = {}
    for r in range(len(qo) - 1):
        n_q, L = int(qo[r + 1] - qo[r]), int(lens[r])
        if n_q == 0 or L == 0:
            continue
        diag = L - n_q
        S = float(np.log(max(L, 2))) + margin
        gamma = S / (beta * sm)
        bounds = [p for p in segment_boundaries(plan_blob, plan, r, L, segments)
                  if p < max(diag, 1)]
        words = _tree_words(b, r) if mode == "tree" else None
        for h in range(Hkv):
            tgt = []
            for t in range(n_q):
                for j in range(g):
                    role = (t * g + j) % 4
                    p = None
                    if mode == "streaming" and L > sink + window + 1:
                        p = [diag + t, L - window - 1, L - window, max(sink - 1, 0)][role]
                    elif role == 0:
                        if mode == "tree":
                            anc = [c for c in range(n_q) if (int(words[t]) >> c) & 1]
                            p = diag + int(rng.choice(anc))
                        elif mode == "none":
                            p = int(rng.integers(0, L))
                        else:
                            p = diag + t
                    elif role == 1:
                        if mode == "tree":
                            hid = [c for c in range(n_q) if not (int(words[t]) >> c) & 1]
                            p = diag + int(rng.choice(hid)) if hid else None
                        elif mode == "causal" and t < n_q - 1:
                            p = diag + t + 1
                    elif role == 2 and bounds:
                        p = int(rng.choice(bounds))
                    if p is None:  # role 3, or no candidate for the others
                        hi = max(diag // TILE, 1)
                        m = int(rng.integers(1, hi + 1)) if diag >= TILE else 0
                        p = min(max(m * TILE - int(rng.integers(0, 2)), 0), L - 1)
                    if mode == "streaming" and role != 1 and not (p < sink or p >= L - window):
                        p = L - 1 - int(rng.integers(0, min(window, L)))
                    tgt.append(p)
                    targets[(r, h, t * g + j)] = p
            pos = sorted(set(tgt))
            basis, _ = np.linalg.qr(rng.standard_normal((D, len(pos))))
            u = {p: basis[:, i] for i, p in enumerate(pos)}
            for p in pos:
                k_pages.append(idx[kvp[r] + p // ps])
                k_slots.append(p % ps)
                k_heads.append(h)
                k_vals.append(gamma * u[p])
            for row, p in enumerate(tgt):
                t, j = divmod(row, g)
                q_rows.append(qo[r] + t)
                q_heads.append(h * g + j)
                q_vals.append(beta * u[p])
    if not q_rows:
        return targets
    qr = torch.from_numpy(np.array(q_rows)).to(dev)
    qh = torch.from_numpy(np.array(q_heads)).to(dev)
    qv = torch.from_numpy(np.array(q_vals, np.float32)).to(dev)
    cur = b.q[qr, qh].float()
    # project the planted directions out of the rows' noise, then add beta * u
    un = qv / beta
    cur = cur - (cur * un).sum(-1, keepdim=True) * un
    b.q[qr, qh] = (cur + qv).to(b.q.dtype)
    kp = torch.from_numpy(np.array(k_pages)).to(dev)
    ks = torch.from_numpy(np.array(k_slots)).to(dev)
    kh = torch.from_numpy(np.array(k_heads)).to(dev)
    kv = torch.from_numpy(np.array(k_vals, np.float32)).to(dev)
    b.cache[kp, 0, ks, kh] = kv.to(b.cache.dtype)
    return targets


def _visibility(mode, n_q, L, words=None, sink=0, window=0, mutate=None):
    if mutate == "nomask":
        vis = np.ones((n_q, L), bool)
    elif mode == "tree":
        blk = ((words[:, None] >> np.arange(n_q, dtype=np.uint64)) & 1).astype(bool)
        vis = np.concatenate([np.ones((n_q, L - n_q), bool), blk], 1)
    else:
        vis = OA.visibility(mode, n_q, L, sink=sink, window=window)
    if mutate == "droplast" and L > 0:
        vis = vis.copy()
        vis[:, ((L - 1) // TILE) * TILE:] = False
    return vis


def oracle_per_request(b, mode="causal", sink=0, window=0, mutations=(), progress=0):
    """fp32 oracle, one request at a time on its own pages gathered on the device.

    Returns {None: (out, lse)} for the reference plus one entry per name in
    `mutations` ("nomask": every token visible; "droplast": each request's last kv
    tile hidden), all computed from the same gathered pages."""
    qo = b.qo_indptr.cpu().numpy().astype(np.int64)
    kvp = b.kv_indptr.cpu().numpy().astype(np.int64)
    lens = b.kv_lens
    nnz = b.q.shape[0]
    ps = b.page_size
    variants = (None,) + tuple(mutations)
    res = {v: (np.zeros((nnz, b.num_qo_heads, b.head_dim), np.float32),
               np.full((nnz, b.num_qo_heads), -np.inf, np.float32)) for v in variants}
    B = len(qo) - 1
    for r in range(B):
        if progress and r % progress == 0:
            say(f"  oracle: request {r}/{B}")
        n_q, L = int(qo[r + 1] - qo[r]), int(lens[r])
        if n_q == 0 or L == 0:
            continue
        pages = b.kv_indices[int(kvp[r]): int(kvp[r + 1])].long()
        sub = b.cache[pages].float().cpu().numpy()
        q = b.q[int(qo[r]): int(qo[r + 1])].float().cpu().numpy()
        n_pages = sub.shape[0]
        last = np.array([L - (n_pages - 1) * ps], np.int32)
        words = _tree_words(b, r) if mode == "tree" else None
        for v in variants:
            vis = _visibility(mode, n_q, L, words, sink, window, v)
            o, l = OA.verify_attention(q, sub, [0, n_q], [0, n_pages],
                                       np.arange(n_pages, dtype=np.int32), last, ps,
                                       mode="custom", custom_mask=vis.ravel(), return_lse=True)
            res[v][0][qo[r]: qo[r + 1]] = o
            res[v][1][qo[r]: qo[r + 1]] = l
    return res
