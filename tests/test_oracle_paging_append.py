"""Pins oracle/paging.py to the reference's known-answer examples and oracle/append.py to
exact scatter/gather identities."""
import numpy as np
import pytest

from oracle import append as OAp
from oracle import attention as OA
from oracle import paging as OP


def test_page_manager_known_answers():
    # batchspec/backends/utils/paging.py:89-129 (B=2, max 64 pages per request)
    pm = OP.Pages(2, 64, 16)
    assert pm.allocate([1, 1]) == [0, 64]
    indptr, indices, _ = pm.table()
    np.testing.assert_array_equal(indptr, [0, 1, 2])
    np.testing.assert_array_equal(indices, [0, 64])
    pm.allocate([1, 0])
    indptr, indices, _ = pm.table()
    np.testing.assert_array_equal(indptr, [0, 2, 3])
    np.testing.assert_array_equal(indices, [0, 1, 64])
    pm.free([1, 0])
    indptr, indices, _ = pm.table()
    np.testing.assert_array_equal(indptr, [0, 1, 2])
    np.testing.assert_array_equal(indices, [0, 64])
    pm.allocate([2, 1])
    assert [len(p) for p in pm.pages] == [3, 2]


def test_page_manager_errors():
    pm = OP.Pages(2, 2, 16)
    pm.allocate([2, 0])
    with pytest.raises(RuntimeError, match="exceed"):
        pm.allocate([1, 0])
    with pytest.raises(RuntimeError, match="more pages than allocated"):
        pm.free([0, 1])


def test_insert_delete_track_token_counts():
    rng = np.random.default_rng(0)
    pm = OP.Pages(3, 512, 16)
    pm.clear_kv()
    tokens = np.zeros(3, dtype=np.int64)
    for _ in range(200):
        if rng.random() < 0.6:
            d = rng.integers(0, 40, size=3)
            pm.insert_kv(d)
            tokens += d
        else:
            d = np.minimum(rng.integers(0, 30, size=3), tokens)
            pm.delete_kv(d)
            tokens -= d
        for r in range(3):
            assert pm.total(r) == tokens[r]
            assert len(pm.pages[r]) == max(1, -(-tokens[r] // 16))
            assert pm.pages[r] == [r * 512 + i for i in range(len(pm.pages[r]))]


def test_append_positions_known_answer():
    # two requests holding 10 and 3 tokens after insert, appending 2 and 3 tokens
    indptr = np.array([0, 1, 2])
    last = np.array([10, 3])
    sl = OA.seq_lens(indptr, last, 16)
    np.testing.assert_array_equal(sl, [10, 3])
    bidx, pos = OAp.get_batch_indices_positions([0, 2, 5], sl, 5)
    np.testing.assert_array_equal(bidx, [0, 0, 1, 1, 1])
    np.testing.assert_array_equal(pos, [8, 9, 0, 1, 2])


def test_append_then_gather_roundtrip_and_untouched_slots():
    rng = np.random.default_rng(1)
    ps, H, D = 4, 2, 8
    ctx = np.array([5, 0, 9])
    n = np.array([3, 2, 4])
    kv = ctx + n
    pages = -(-kv // ps)
    indptr = np.concatenate([[0], np.cumsum(pages)])
    P = int(indptr[-1]) + 3
    idx = rng.permutation(P)[: indptr[-1]]
    last = (kv - 1) % ps + 1
    cache = rng.normal(size=(P, 2, ps, H, D)).astype(np.float32)
    ap = np.concatenate([[0], np.cumsum(n)])
    k = rng.normal(size=(int(ap[-1]), H, D)).astype(np.float32)
    v = rng.normal(size=(int(ap[-1]), H, D)).astype(np.float32)
    out = OAp.update(k, v, ap, cache, indptr, idx, last, ps)
    written = np.zeros(cache.shape[:3], dtype=bool)
    for b in range(3):
        K, V = OA.gather_kv(out, indptr, idx, ps, b, int(kv[b]))
        np.testing.assert_array_equal(K[ctx[b]:], k[ap[b]:ap[b + 1]])
        np.testing.assert_array_equal(V[ctx[b]:], v[ap[b]:ap[b + 1]])
        K0, _ = OA.gather_kv(cache, indptr, idx, ps, b, int(kv[b]))
        np.testing.assert_array_equal(K[:ctx[b]], K0[:ctx[b]])
        pg, sl = OA.token_slots(indptr, idx, ps, b, int(kv[b]))
        written[pg[ctx[b]:], :, sl[ctx[b]:]] = True
    np.testing.assert_array_equal(out[~written], cache[~written])
