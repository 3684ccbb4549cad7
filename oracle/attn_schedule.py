"""ORACLE — TEST INFRASTRUCTURE ONLY.  CPU restatement of the device-side attention
schedule (bsx_attn_plan_device) and of the invariants every schedule must satisfy.

The reference has no device-side planner (FlashInfer's plan() schedules on the host,
batchspec/backends/base/attn_wrapper.py:33-72); what a schedule must do for the
attention to be the reference's is fixed by its inputs:
  * kv_len = (pages - 1) * page_size + last_page_len (get_seq_lens,
    batchspec/models/modules/kv_cache.py:66-70), seq record {qo_start, qo_len,
    kv_len, page_start};
  * every kv tile of every request with query tokens is attended exactly once
    (the sink+window view: only the sink tiles and the window tiles), and a request
    with query tokens but no kv still gets one (empty) segment so its output is
    written;
  * a request cut into several segments gets one partial slot per segment and one
    merge record.
`schedule` restates the equal-share cut of the device planner (same integer
arithmetic); `check_invariants` checks any blob against the properties above, so the
restatement itself is pinned by them and by the attention results the schedule yields.
"""
from __future__ import annotations

import numpy as np

TILE = 32
SEG_COST = 2
ERR_INVALID = -1
ERR_UNSUPPORTED = -3
MASK_STREAMING = 3


def units_of(qlen: int, kl: int, mask_mode: int, sink: int, window: int):
    """Tile ranges [(begin, end), ...] of one request's work units."""
    if qlen == 0:
        return []
    nt = (kl + TILE - 1) // TILE
    if mask_mode == MASK_STREAMING and kl > sink + window:
        a_end = (sink + TILE - 1) // TILE
        w_beg = max(0, kl - window) // TILE
        if w_beg <= a_end:
            return [(0, nt)]
        if a_end > 0:
            return [(0, a_end), (w_beg, nt)]
        return [(w_beg, nt)]
    return [(0, nt)]


def layout(B: int, W: int):
    """Offsets of bsx_attn_plan_device_shape's blob layout."""
    max_segs = W + 2 * B
    off_seg_indptr = 4 * B
    off_segments = off_seg_indptr + W + 1
    off_merge = (off_segments + 4 * max_segs + 3) & ~3
    off_part = off_merge + 4 * B
    off_dyn = off_part + B + 1
    return dict(off_seg_indptr=off_seg_indptr, off_segments=off_segments, off_merge=off_merge,
                off_part=off_part, off_dyn=off_dyn, ints=off_dyn + 4, max_segs=max_segs)


def schedule(qo_indptr, kv_indptr, last, page_size: int, mask_mode: int, sink: int, window: int,
             max_qo: int, W: int, kv_indices_len: int = -1):
    """Expected blob entries: dict of the written parts (unwritten slots are not compared)."""
    qo = np.asarray(qo_indptr, np.int64)
    kvp = np.asarray(kv_indptr, np.int64)
    last = np.asarray(last, np.int64)
    B = len(qo) - 1
    err = 0
    seq = []
    for b in range(B):
        q0, q1, p0, p1 = qo[b], qo[b + 1], kvp[b], kvp[b + 1]
        np_, qlen = p1 - p0, q1 - q0
        e = 0
        if (b == 0 and (q0 != 0 or p0 != 0)) or qlen < 0 or np_ < 0:
            e = ERR_INVALID
        if last[b] < 0 or last[b] > page_size:
            e = ERR_INVALID
        if qlen > max_qo:
            e = ERR_UNSUPPORTED
        kl = (np_ - 1) * page_size + last[b] if np_ > 0 else 0
        if kl >= (1 << 30):
            e = ERR_UNSUPPORTED
        err = min(err, e)  # the most negative code of all violations
        seq.append((int(q0), 0 if e else int(qlen), 0 if e else int(kl), int(p0)))
    if kvp[B] < 1 or (kv_indices_len >= 0 and kvp[B] > kv_indices_len):
        err = min(err, ERR_INVALID)
    units = [units_of(s[1], s[2], mask_mode, sink, window) for s in seq]
    cpre, c = [], 0
    for us in units:
        cpre.append(c)
        c += sum(max(1, e - b) + SEG_COST for b, e in us)
    T = 0 if err else c
    Wn = min(W, T)
    wg = lambda pos: ((pos + 1) * Wn - 1) // T
    sbeg = lambda w: w * T // Wn
    segs, seg_wg, part, merge = [], [], [], []
    npart = 0
    for b in range(B):
        pieces = []
        if T > 0:
            s = cpre[b]
            for tb, te in units[b]:
                n = te - tb
                p = s + SEG_COST
                wf = wg(p)
                wl = wg(p + n - 1) if n > 0 else wf
                for w in range(wf, wl + 1):
                    lo, hi = max(sbeg(w), p), min(sbeg(w + 1), p + n)
                    pieces.append((b, tb + (lo - p) if n else tb, tb + (hi - p) if n else tb, w))
                s += max(1, n) + SEG_COST
        split = len(pieces) > 1
        part.append(npart)
        if split:
            merge.append((npart, npart + len(pieces), seq[b][0], seq[b][1]))
        for k, (bb, t0, t1, w) in enumerate(pieces):
            segs.append((bb, t0, t1, npart + k if split else -1))
            seg_wg.append(w)
        if split:
            npart += len(pieces)
    part.append(npart)
    seg_indptr = [sum(1 for w in seg_wg if w < x) if x < Wn else len(segs) for x in range(W + 1)]
    return dict(seq=np.array(seq, np.int32).reshape(-1, 4), seg_indptr=np.array(seg_indptr, np.int32),
                segments=np.array(segs, np.int32).reshape(-1, 4),
                merge=np.array(merge, np.int32).reshape(-1, 4), part=np.array(part, np.int32),
                dyn=np.array([len(merge), err, len(segs), 0], np.int32))


def read_blob(blob: np.ndarray, B: int, W: int):
    """The written parts of a device blob, as `schedule` returns them."""
    L = layout(B, W)
    dyn = blob[L["off_dyn"]: L["off_dyn"] + 4].copy()
    nseg, M = int(dyn[2]), int(dyn[0])
    return dict(seq=blob[: 4 * B].reshape(-1, 4).copy(),
                seg_indptr=blob[L["off_seg_indptr"]: L["off_seg_indptr"] + W + 1].copy(),
                segments=blob[L["off_segments"]: L["off_segments"] + 4 * nseg].reshape(-1, 4).copy(),
                merge=blob[L["off_merge"]: L["off_merge"] + 4 * M].reshape(-1, 4).copy(),
                part=blob[L["off_part"]: L["off_part"] + B + 1].copy(), dyn=dyn)


def check_invariants(s, qo_indptr, kv_indptr, last, page_size: int, mask_mode: int, sink: int,
                     window: int):
    """Schedule properties the attention's correctness rests on (raises AssertionError)."""
    qo = np.asarray(qo_indptr, np.int64)
    B = len(qo) - 1
    if s["dyn"][1] != 0:
        assert len(s["segments"]) == 0 and (s["seg_indptr"] == 0).all()
        return
    kl = [(kv_indptr[b + 1] - kv_indptr[b] - 1) * page_size + last[b]
          if kv_indptr[b + 1] > kv_indptr[b] else 0 for b in range(B)]
    for b in range(B):
        assert tuple(s["seq"][b]) == (qo[b], qo[b + 1] - qo[b], kl[b], kv_indptr[b])
    sp = s["seg_indptr"]
    assert sp[0] == 0 and (np.diff(sp) >= 0).all() and sp[-1] == len(s["segments"])
    covered = {b: [] for b in range(B)}
    slots = {b: [] for b in range(B)}
    for b, t0, t1, slot in s["segments"]:
        assert t0 <= t1
        covered[b].append((t0, t1))
        slots[b].append(slot)
    for b in range(B):
        want = units_of(int(qo[b + 1] - qo[b]), int(kl[b]), mask_mode, sink, window)
        got = sorted(covered[b])
        tiles = sorted(t for t0, t1 in got for t in range(t0, t1))
        assert tiles == sorted(t for tb, te in want for t in range(tb, te)), b
        if want and not tiles:
            assert len(got) >= 1  # empty request still has its output segment
        if len(slots[b]) > 1:
            assert sorted(slots[b]) == list(range(s["part"][b], s["part"][b + 1]))
        else:
            assert all(x == -1 for x in slots[b]) and s["part"][b + 1] == s["part"][b]
    split = [b for b in range(B) if len(slots[b]) > 1]
    assert s["dyn"][0] == len(split) == len(s["merge"])
    for m, b in zip(s["merge"], split):
        assert tuple(m) == (s["part"][b], s["part"][b + 1], qo[b], qo[b + 1] - qo[b])
