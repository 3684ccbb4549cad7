"""Accepted-KV compaction oracle, pinned by the known answer in the docstring of
batchspec/backends/mtp_engine.py:589-593 and by the invariants that define the move."""
import numpy as np

from oracle import collate as OC


def test_docstring_known_answer():
    # k=3, accept_nums=[2, 3], prev_cachelens=[10, 15] (mtp_engine.py:589-593)
    save = OC.save_indices([2, 3], [10, 15], 3)
    assert save == [[10, 14], [15, 19, 23]]
    # the docstring's delete indices: the k(k+1) inserted positions minus the saved ones
    k = 3
    delete = [[p for p in range(prev, prev + k * (k + 1)) if p not in s]
              for prev, s in zip([10, 15], save)]
    assert delete == [[11, 12, 13, 15, 16, 17, 18, 19, 20, 21],
                      [16, 17, 18, 20, 21, 22, 24, 25, 26]]


def _batch(rng, B, k, ps, H, D, pages_per_req=8):
    P = B * pages_per_req + 3
    perm = rng.permutation(P)[: B * pages_per_req].astype(np.int32)
    indptr = np.arange(B + 1, dtype=np.int32) * pages_per_req
    prev = rng.integers(0, pages_per_req * ps - (k + 1) ** 2, size=B).astype(np.int32)
    acc = rng.integers(1, k + 2, size=B).astype(np.int64)
    cache = rng.standard_normal((P, 2, ps, H, D)).astype(np.float32)
    return cache, acc, prev, indptr, perm


def _logical(cache, indptr, indices, ps, b, n):
    pos = np.arange(n)
    return cache[indices[indptr[b] + pos // ps], :, pos % ps]


def test_moves_exactly_the_accepted_rows():
    rng = np.random.default_rng(3)
    k, ps = 4, 16
    cache, acc, prev, indptr, idx = _batch(rng, 6, k, ps, 2, 8)
    out = OC.collate(cache, acc, prev, k, indptr, idx, ps)
    n = 8 * ps
    for b in range(6):
        before = _logical(cache, indptr, idx, ps, b, n)
        after = _logical(out, indptr, idx, ps, b, n)
        for i in range(int(acc[b])):
            np.testing.assert_array_equal(after[prev[b] + i], before[prev[b] + i * (k + 1)])
        others = [p for p in range(n) if not (prev[b] <= p < prev[b] + acc[b])]
        np.testing.assert_array_equal(after[others], before[others])
    # pages no request owns stay as they were
    free = np.setdiff1d(np.arange(cache.shape[0]), idx)
    np.testing.assert_array_equal(out[free], cache[free])


def test_page_permutation_invariance():
    rng = np.random.default_rng(4)
    k, ps = 3, 8
    cache, acc, prev, indptr, idx = _batch(rng, 4, k, ps, 2, 4)
    out = OC.collate(cache, acc, prev, k, indptr, idx, ps)
    # the same logical cache laid out contiguously (the reference's own layout)
    n = 8 * ps
    contig = np.stack([_logical(cache, indptr, idx, ps, b, n) for b in range(4)])  # [B, n, 2, H, D]
    flat = contig.reshape(4 * 8, ps, 2, 2, 4).transpose(0, 2, 1, 3, 4)  # pages [P, 2, ps, H, D]
    cidx = np.arange(4 * 8, dtype=np.int32)
    cout = OC.collate(flat, acc, prev, k, indptr, cidx, ps)
    for b in range(4):
        np.testing.assert_array_equal(_logical(out, indptr, idx, ps, b, n),
                                      _logical(cout, indptr, cidx, ps, b, n))
