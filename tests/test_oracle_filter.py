"""Top-k / top-p renormalisation, sample() and filtered acceptance of the CPU oracle
(oracle/filter.c), pinned by:
  * a float64 restatement of the reference's order (batchspec/backends/utils/sampling.py:
    48-56: softmax, then top-p on the full distribution, then top-k on the
    renormalised one) on random rows, away from rounding ties at the nucleus edge;
  * known answers where that order matters and where ties sit at the threshold;
  * the identity cases (filters off), the draw's comparison direction and index order,
  * the distribution of sample() under stratified uniforms, and the speculative-sampling
    guarantee (the first emitted token is distributed as the filtered target) by a
    chi-square test."""
import math

import numpy as np
import pytest

from oracle import accept as A


def _ref_filtered(x, T, top_k, top_p):
    """float64 restatement of sampling.py:48-56 with threshold (pivot) semantics."""
    z = x.astype(np.float64) / T
    p = np.exp(z - z.max())
    p /= p.sum()
    if 0 < top_p < 1:
        order = np.sort(p)[::-1]
        c = np.cumsum(order)
        i = int(np.argmax(c >= top_p)) if (c >= top_p).any() else len(p) - 1
        pivot = order[i]
        p = np.where(p >= pivot, p, 0.0)
        p /= p.sum()
    if 0 < top_k < len(p):
        pivot = np.sort(p)[::-1][top_k - 1]
        p = np.where(p >= pivot, p, 0.0) if pivot > 0 else p
        p /= p.sum()
    return p


def _nucleus_margin(x, T, top_p):
    z = x.astype(np.float64) / T
    p = np.exp(z - z.max())
    p /= p.sum()
    c = np.cumsum(np.sort(p)[::-1])
    return np.min(np.abs(c - top_p))


@pytest.mark.parametrize("T,top_k,top_p", [(1.0, 20, 0.95), (0.6, 20, 0.95), (1.0, 0, 0.9),
                                            (1.0, 50, 0.0), (0.7, 5, 0.3), (1.3, 200, 0.99)])
def test_matches_float64_restatement(T, top_k, top_p):
    rng = np.random.default_rng(11)
    V = 3000
    checked = 0
    for r in range(12):
        x = (rng.standard_normal(V) * (1.0 + r % 3)).astype(np.float32)
        if 0 < top_p < 1 and _nucleus_margin(x, T, top_p) < 3e-6:
            continue
        want = _ref_filtered(x, T, top_k, top_p)
        got = A.filtered_probs(x[None], T, top_k, top_p)[0]
        np.testing.assert_array_equal(got > 0, want > 0)
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-9)
        checked += 1
    assert checked >= 8


def test_reference_order_known_answer():
    # probs [0.4, 0.3, 0.2, 0.1]: top-p 0.5 on the full distribution keeps {0.4, 0.3}, then
    # top-k 2 keeps both: [4/7, 3/7].  (top-k first would renormalise to [4/7, 3/7] and the
    # nucleus 0.5 would then keep only the first token.)
    x = np.log(np.array([0.4, 0.3, 0.2, 0.1], np.float64)).astype(np.float32)
    got = A.filtered_probs(x[None], 1.0, 2, 0.5)[0]
    np.testing.assert_allclose(got, [4 / 7, 3 / 7, 0, 0], rtol=1e-5)
    np.testing.assert_allclose(A.filtered_probs(x[None], 1.0, 1, 0.5)[0], [1, 0, 0, 0], rtol=1e-6)
    np.testing.assert_allclose(A.filtered_probs(x[None], 1.0, 0, 0.35)[0], [1, 0, 0, 0], rtol=1e-6)
    np.testing.assert_allclose(A.filtered_probs(x[None], 1.0, 3, 0.0)[0],
                               [4 / 9, 3 / 9, 2 / 9, 0], rtol=1e-5)


def test_ties_at_threshold_are_kept():
    x = np.array([5, 5, 5, 1, 0, -2, 5.5], np.float32)
    got = A.filtered_probs(x[None], 1.0, 2, 0.0)[0]
    assert np.all(got[[0, 1, 2, 6]] > 0) and np.all(got[[3, 4, 5]] == 0)
    e = math.exp(0.5)
    np.testing.assert_allclose(got[[6, 0]], [e / (e + 3), 1 / (e + 3)], rtol=1e-5)
    # the same threshold whatever the order of the row
    perm = np.random.default_rng(1).permutation(len(x))
    np.testing.assert_array_equal(A.filtered_probs(x[perm][None], 1.0, 2, 0.0)[0], got[perm])


@pytest.mark.parametrize("top_k,top_p", [(0, 1.0), (0, 0.0), (-3, 1.5), (1000, 1.0), (1001, 0.0)])
def test_filters_off_is_plain_softmax(top_k, top_p):
    x = (np.random.default_rng(2).standard_normal((3, 1000)) * 2).astype(np.float32)
    np.testing.assert_array_equal(A.filtered_probs(x, 0.8, top_k, top_p), A.softmax(x, 0.8))


def test_draw_direction_and_order():
    r = np.array([0, 0.25, 0, 0.5, 0.25], np.float32)  # fixed point: [0, 2^38, 0, 2^39, 2^38]
    assert A.fx_draw(r, 0.0) == 1
    assert A.fx_draw(r, np.nextafter(np.float32(0.25), np.float32(0))) == 1
    assert A.fx_draw(r, 0.25) == 3          # running sum must exceed the point
    assert A.fx_draw(r, 0.75) == 4
    assert A.fx_draw(r, np.nextafter(np.float32(1), np.float32(0))) == 4
    assert A.fx_draw(r, -1.0) == 1          # non-positive uniforms draw the first token
    assert A.fx_draw(np.zeros(4, np.float32), 0.5) == -1


def test_u64_to_f32_rounds_to_nearest_even():
    assert A.u64_to_f32(2**24 + 1) == 2.0**24          # tie -> even
    assert A.u64_to_f32(2**24 + 3) == 2.0**24 + 4      # tie -> even (up)
    assert A.u64_to_f32(2**40 + 2**16 + 1) == np.float32(2**40 + 2**17)
    assert A.u64_to_f32(12345) == 12345.0
    rng = np.random.default_rng(3)
    # below 2^53 the conversion through binary64 is exact, so numpy's float32 is the answer
    for v in rng.integers(0, 2**53, size=200, dtype=np.uint64):
        assert A.u64_to_f32(int(v)) == float(np.float32(float(int(v))))


def test_sample_stratified_frequencies():
    x = np.array([2.0, 1.5, 1.4, 0.3, -1.0, 1.5, 0.9, -3.0], np.float32)
    N = 4000
    u = ((np.arange(N) + 0.5) / N).astype(np.float32)
    for T, k, p in [(1.0, 4, 0.9), (0.6, 0, 0.8), (1.0, 3, 1.0)]:
        want = A.filtered_probs(x[None], T, k, p)[0].astype(np.float64)
        got = A.sample(np.repeat(x[None], N, 0), T, k, p, u)
        freq = np.bincount(got, minlength=len(x)) / N
        np.testing.assert_allclose(freq, want, atol=1.5 / N)


def test_chain_emits_the_filtered_target_distribution():
    # Leviathan et al. 2023: the first emitted token ~ p' when the draft token ~ q'.
    rng = np.random.default_rng(5)
    V, N, T, k_top, p_top = 7, 60000, 1.0, 4, 0.9
    t = (rng.standard_normal((2, V)) * 1.5).astype(np.float32)
    d = (t[:1] + rng.standard_normal((1, V)).astype(np.float32)).astype(np.float32)
    draft_tok = A.sample(np.repeat(d, N, 0), T, k_top, p_top, rng.random(N, dtype=np.float32))
    u = rng.random((N, 2), dtype=np.float32)
    out, acc, emi = A.chain_filtered(np.repeat(d[None], N, 0), draft_tok[:, None],
                                     np.repeat(t[None], N, 0), T, k_top, p_top, u)
    p0 = A.filtered_probs(t[:1], T, k_top, p_top)[0].astype(np.float64)
    obs = np.bincount(out[:, 0], minlength=V)
    assert np.all(obs[p0 == 0] == 0)
    m = p0 > 0
    chi2 = float((((obs[m] - N * p0[m]) ** 2) / (N * p0[m])).sum())
    # df = m.sum() - 1 <= 3: the 0.999 quantile of chi2(3) is 16.3
    assert chi2 < 16.3, (chi2, obs, N * p0)
    assert np.all(emi <= 1) and np.all(acc == emi)


def test_filters_off_matches_unfiltered_chain():
    rng = np.random.default_rng(6)
    B, k, V = 5, 3, 500
    t = rng.standard_normal((B, k + 1, V)).astype(np.float32)
    d = rng.standard_normal((B, k, V)).astype(np.float32)
    ids = rng.integers(0, V, size=(B, k))
    u = rng.random((B, k + 1), dtype=np.float32)
    for dl in (None, d):
        a = A.chain_filtered(dl, ids, t, 0.9, 0, 1.0, u)
        b = A.chain_logits(dl, ids, t, 0.9, u)
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)


def test_one_hot_draft_of_argmax_with_top1_always_accepts():
    rng = np.random.default_rng(7)
    B, k, V = 6, 4, 300
    t = rng.standard_normal((B, k + 1, V)).astype(np.float32)
    ids = t[:, :k].argmax(-1)
    u = rng.random((B, k + 1), dtype=np.float32)
    out, acc, emi = A.chain_filtered(None, ids, t, 1.0, 1, 0.0, u)
    assert np.all(emi == k) and np.all(acc == k)
    np.testing.assert_array_equal(out[:, k], t[:, k].argmax(-1))
