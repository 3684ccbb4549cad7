"""Pins the acceptance oracle (oracle/accept.py, oracle/accept.c) against libm, float64
references, hand-computed known answers and the speculative-sampling invariant."""
import math

import numpy as np
import pytest
import torch

from oracle import accept as A


# ---------------------------------------------------------------- exp2 / softmax
def test_exp2_within_3e6_of_libm(oracle_lib):
    # the degree-4 polynomial's worst case on [0, 1) is 2.96e-6 relative (y - floor(y)
    # and the ldexp are exact for these arguments); a dropped or perturbed coefficient
    # moves it far beyond the bound
    ys = np.concatenate([np.linspace(-125.0, 0.0, 500001, dtype=np.float32),
                         np.float32(-np.random.default_rng(0).random(20000) * 30)])
    got = A.exp2_array(ys).astype(np.float64)
    ref = np.exp2(ys.astype(np.float64))
    rel = np.abs(got - ref) / ref
    assert rel.max() <= 3.0e-6
    assert rel.max() >= 2.0e-6  # the fit's own error is reached: it is degree 4
    # monotone in y across the integer steps of the argument
    yy = np.sort(np.float32(-np.random.default_rng(5).random(200000) * 8))
    assert np.all(np.diff(A.exp2_array(yy).astype(np.float64)) >= 0)
    assert A.exp2(0.0) == 1.0
    assert A.exp2(-1.0) == 0.5
    assert A.exp2(-300.0) == 0.0
    # no clamp: far below the float range, beyond int32 and -inf all underflow to 0
    assert A.exp2(-1e30) == 0.0 and A.exp2(-3e9) == 0.0 and A.exp2(float("-inf")) == 0.0
    # denormal results round like ldexp
    assert A.exp2(-149.0) == 2.0 ** -149
    assert A.exp2(-127.5) == float(np.ldexp(np.float32(A.exp2(0.5)), -128))


@pytest.mark.parametrize("T", [1.0, 0.6, 1.7])
def test_softmax_close_to_float64(T):
    x = np.random.default_rng(1).normal(0, 3, size=(4, 3001)).astype(np.float32)
    p = A.softmax(x, T).astype(np.float64)
    y = x.astype(np.float64) / T
    r = np.exp(y - y.max(-1, keepdims=True))
    r /= r.sum(-1, keepdims=True)
    # C = log2(e)/T is a binary32 constant (relative error <= 1.5e-7), so the error of
    # an exponent grows with its distance from the row max: bound 2e-7 per bit of
    # log2-distance plus the exp2's 3e-6 (on the weight and on Z) and the sum's rounding.
    bits = -np.log2(r) + 1
    assert np.all(np.abs(p - r) / r < 2e-7 * bits + 8e-6)


def test_row_stats_sum_matches_fsum():
    x = np.random.default_rng(2).normal(0, 2, size=50000).astype(np.float32)
    M, Z = A.row_stats(x)
    assert M == x.max()
    c = np.float32(1 / math.log(2))
    w = np.exp2(x.astype(np.float64) * float(c) - float(M) * float(c))
    assert abs(Z - math.fsum(w)) / math.fsum(w) < 4e-6


def test_row_stats_lanes_starting_at_minus_inf():
    # the first two rounds of groups are -inf, so every lane's reference starts from its
    # start value and is rescaled from there (an exact power of two, applied to 0)
    V = 40000
    x = np.random.default_rng(3).normal(0, 2, size=V).astype(np.float32)
    x[: 8 * 2048 * 2] = -np.inf
    M, Z = A.row_stats(x)
    fin = x[np.isfinite(x)].astype(np.float64)
    assert M == fin.max()
    c = np.float32(1 / math.log(2))
    w = np.exp2(fin * float(c) - float(M) * float(c))
    assert abs(Z - math.fsum(w)) / math.fsum(w) < 4e-6


@pytest.mark.parametrize("order", ["ascending", "descending"])
def test_row_stats_rescales_are_exact(order):
    # ascending: every group raises its lane's maximum (a rescale per group); descending:
    # none after the first.  Powers of two are exact, so only exp2 and the sums round.
    x = np.sort(np.random.default_rng(4).normal(0, 4, size=60000).astype(np.float32))
    if order == "descending":
        x = x[::-1].copy()
    M, Z = A.row_stats(x)
    c = np.float32(1 / math.log(2))
    w = np.exp2(x.astype(np.float64) * float(c) - float(M) * float(c))
    assert M == x.max()
    assert abs(Z - math.fsum(w)) / math.fsum(w) < 4e-6


@pytest.mark.parametrize("scale", [1e3, 1e6, 1e8])
def test_softmax_large_logits_within_domain(scale):
    # |x * C| < 2^31: a weight's exponent is at most the rounding error of fl(x * C)
    # (here up to 32), so Z stays finite and the probabilities sum to 1
    x = (np.random.default_rng(5).normal(0, 1, size=(2, 5000)) * scale).astype(np.float32)
    assert np.abs(x).max() * 1.4427 < 2.0 ** 31
    p = A.softmax(x)
    assert np.all(np.isfinite(p))
    assert np.all(np.abs(p.sum(-1) - 1.0) < 1e-5)


def test_masked_logits_have_zero_probability():
    x = np.array([0.0, -np.inf, 1.0, -1e30, 2.0], dtype=np.float32)
    p = A.softmax(x[None])[0]
    assert p[1] == 0.0 and p[3] == 0.0
    assert abs(p.sum() - 1) < 1e-6


# ---------------------------------------------------------------- tree draw
def _canonical_order(V):
    """Element order of the canonical tree: lane (8t+i) owns groups t+256i+2048j."""
    G = (V + 7) // 8
    order = []
    for lam in range(2048):
        t, i = lam >> 3, lam & 7
        g = t + 256 * i
        while g < G:
            order.extend(range(8 * g, min(8 * g + 8, V)))
            g += 2048
    return np.array(order)


@pytest.mark.parametrize("V", [7, 1000, 40000])
def test_tree_draw_equals_float64_linear_scan(V):
    rng = np.random.default_rng(V)
    order = _canonical_order(V)
    assert sorted(order.tolist()) == list(range(V))
    checked = 0
    for trial in range(60):
        w = rng.random(V).astype(np.float32) * (rng.random(V) < 0.3)
        if w.sum() == 0:
            continue
        u = float(np.float32(rng.random()))
        got = A.tree_draw(w, u)
        cdf = np.cumsum(w[order].astype(np.float64))
        target = u * cdf[-1]
        pos = int(np.searchsorted(cdf, target, side="right"))
        # skip draws within float32 rounding of a bucket edge
        edges = np.array([cdf[pos - 1] if pos > 0 else 0.0, cdf[min(pos, len(cdf) - 1)]])
        if np.min(np.abs(edges - target)) < 1e-5 * cdf[-1]:
            continue
        assert got == order[pos], (trial, got, order[pos])
        assert w[got] > 0
        checked += 1
    assert checked > 30


# ---------------------------------------------------------------- chain sampling
def test_equal_distributions_accept_everything():
    rng = np.random.default_rng(3)
    B, k, V = 16, 4, 50
    p = rng.dirichlet(np.ones(V), size=(B, k + 1)).astype(np.float32)
    q = p[:, :k].copy()
    ids = rng.integers(0, V, size=(B, k))
    u = rng.random((B, k + 1)).astype(np.float32)
    out, acc, emi = A.chain_probs(q, ids, p, u)
    ok = p[np.arange(B)[:, None], np.arange(k)[None], ids] > 0
    assert np.all(emi[ok.all(1)] == k)
    assert np.all(out[:, :k][ok.all(1)] == ids[ok.all(1)])


def test_disjoint_support_rejects_and_draws_residual():
    B, k, V = 3, 2, 10
    p = np.zeros((B, k + 1, V), np.float32)
    q = np.zeros((B, k, V), np.float32)
    p[:, :, 7] = 1.0
    q[:, :, 2] = 1.0
    ids = np.full((B, k), 2)
    u = np.array([[0.0, 0.5, 0.3], [0.9, 0.1, 0.99], [0.5, 0.5, 0.0]], np.float32)
    out, acc, emi = A.chain_probs(q, ids, p, u)
    np.testing.assert_array_equal(emi, [0, 0, 0])
    np.testing.assert_array_equal(acc, [0, 0, 0])
    np.testing.assert_array_equal(out, [[7, -1, -1]] * 3)


def test_known_answer_small_chain():
    # p0 = [.5,.5], q0 = [1,0], draft 0: u=.4 -> .4*1 < .5 accept; p1=[.2,.8], q1=[0,1],
    # draft 1: u=.9 -> .9 >= .8 reject -> residual max(0,p1-q1) = [.2, 0] -> token 0.
    p = np.array([[[0.5, 0.5], [0.2, 0.8], [0.3, 0.7]]], np.float32)
    q = np.array([[[1.0, 0.0], [0.0, 1.0]]], np.float32)
    out, acc, emi = A.chain_probs(q, [[0, 1]], p, [[0.4, 0.9, 0.5]])
    np.testing.assert_array_equal(out, [[0, 0, -1]])
    assert emi[0] == 1 and acc[0] == 1
    # all accepted -> bonus drawn from p2 with u=.5 over cdf [.3, 1.0] -> token 1
    out, acc, emi = A.chain_probs(q, [[0, 1]], p, [[0.4, 0.7, 0.5]])
    np.testing.assert_array_equal(out, [[0, 1, 1]])
    assert emi[0] == 2 and acc[0] == 2


def _chi2_ok(counts, probs, n):
    exp = probs * n
    stat = float(((counts - exp) ** 2 / exp).sum())
    dof = len(probs) - 1
    # 1e-4 tail of chi-square(dof) via the Wilson-Hilferty approximation
    z = 3.719
    crit = dof * (1 - 2 / (9 * dof) + z * math.sqrt(2 / (9 * dof))) ** 3
    return stat < crit, stat, crit


def test_emitted_token_is_distributed_as_target():
    """Speculative sampling invariant (Leviathan et al. 2023; Chen et al. 2023): the first
    emitted token is distributed exactly as p_0, whatever q_0 is."""
    rng = np.random.default_rng(4)
    V, n = 8, 120000
    p0 = np.array([0.30, 0.05, 0.15, 0.02, 0.18, 0.10, 0.12, 0.08], np.float32)
    q0 = np.array([0.05, 0.30, 0.10, 0.20, 0.05, 0.10, 0.10, 0.10], np.float32)
    p1 = np.full(V, 1 / V, np.float32)
    x = rng.choice(V, size=n, p=q0 / q0.sum())
    u = rng.random((n, 2)).astype(np.float32)
    P = np.broadcast_to(np.stack([p0, p1]), (n, 2, V))
    Q = np.broadcast_to(q0, (n, 1, V))
    out, acc, emi = A.chain_probs(Q, x[:, None], P, u)
    counts = np.bincount(out[:, 0], minlength=V).astype(np.float64)
    ok, stat, crit = _chi2_ok(counts, p0.astype(np.float64) / p0.sum(), n)
    assert ok, (stat, crit)
    # acceptance rate = sum min(p, q)
    assert abs((emi == 1).mean() - np.minimum(p0, q0).sum()) < 0.01


def test_logit_path_equals_probability_path_on_canonical_softmax():
    rng = np.random.default_rng(5)
    B, k, V = 6, 3, 300
    tl = rng.normal(0, 2, size=(B, k + 1, V)).astype(np.float32)
    dl = (tl[:, :k] + rng.normal(0, 0.5, size=(B, k, V))).astype(np.float32)
    ids = rng.integers(0, V, size=(B, k))
    u = rng.random((B, k + 1)).astype(np.float32)
    a = A.chain_logits(dl, ids, tl, 0.8, u)
    b = A.chain_probs(A.softmax(dl, 0.8), ids, A.softmax(tl, 0.8), u)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


# ---------------------------------------------------------------- greedy
def test_argmax_matches_torch_semantics():
    x = np.array([[1.0, 3.0, 3.0, 2.0], [np.nan, 1.0, np.nan, 5.0], [-0.0, 0.0, -1.0, 0.0],
                  [-np.inf, -np.inf, -np.inf, -np.inf]], np.float32)
    np.testing.assert_array_equal(A.argmax(x), torch.from_numpy(x).argmax(-1).numpy())
    np.testing.assert_array_equal(A.argmax(x), [1, 0, 0, 0])


def test_greedy_known_answers():
    # draft [a, b, c], target preds [a, x, c, d]: reference rule counts 2 matches (+1 = 3,
    # bonus = preds[2] = c); the prefix rule stops at the first miss (2, bonus = x).
    a, b_, c, d, x = 5, 6, 7, 8, 9
    draft = np.array([[a, b_, c]])
    preds = np.array([[a, x, c, d]])
    bonus, acc, eos = A.greedy_posterior(draft, preds, eos_token_id=c)
    assert acc[0] == 3 and bonus[0, 0] == c and eos[0, 0]
    bonus, acc, eos = A.greedy_posterior(draft, preds, eos_token_id=c, rule="prefix")
    assert acc[0] == 2 and bonus[0, 0] == x and not eos[0, 0]


def test_greedy_exhaustive_tiny():
    V, k = 3, 2
    import itertools
    for dr in itertools.product(range(V), repeat=k):
        for pr in itertools.product(range(V), repeat=k + 1):
            bonus, acc, eos = A.greedy_posterior(np.array([dr]), np.array([pr]), eos_token_id=1)
            m = sum(1 for i in range(k) if dr[i] == pr[i])
            assert acc[0] == m + 1 and bonus[0, 0] == pr[m]
            assert eos[0, 0] == any(dr[i] == 1 and dr[i] == pr[i] for i in range(k))
            n = 0
            while n < k and dr[n] == pr[n]:
                n += 1
            bonus, acc, eos = A.greedy_posterior(np.array([dr]), np.array([pr]), 1, rule="prefix")
            assert acc[0] == n + 1 and bonus[0, 0] == pr[n]
