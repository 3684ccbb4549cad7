"""The oracle against the committed golden fixtures (tests/golden/make_golden.py writes
them from computations independent of the oracle: torch float64 SDPA, direct position
loops, the reference's greedy tensor expressions, a float64 sequential chain rule)."""
from pathlib import Path

import numpy as np
import pytest

from oracle import accept as OAc
from oracle import append as OAp
from oracle import attention as OA

G = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(G / name, allow_pickle=False))


def test_attention_matches_float64_sdpa():
    f = load("config1_attention.npz")
    out, lse = OA.verify_attention(f["q"], f["cache"], f["qo_indptr"], f["kv_indptr"],
                                   f["kv_indices"], f["kv_last_page_len"], int(f["page_size"]),
                                   mode="causal", return_lse=True)
    np.testing.assert_allclose(out, f["out"], atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse, f["lse"], atol=2e-5, rtol=1e-6)


def test_append_writes_exactly_the_golden_slots():
    a = load("config1_attention.npz")
    f = load("config1_append.npz")
    cache = a["cache"]
    new = OAp.update(f["k_new"], f["v_new"], a["qo_indptr"], cache, a["kv_indptr"],
                     a["kv_indices"], a["kv_last_page_len"], int(a["page_size"]))
    P, S = f["target_page"], f["target_slot"]
    np.testing.assert_array_equal(new[P, 0, S], f["k_new"])
    np.testing.assert_array_equal(new[P, 1, S], f["v_new"])
    touched = np.zeros(cache.shape[:3], bool)
    touched[P, :, S] = True
    np.testing.assert_array_equal(new[~touched], cache[~touched])


def test_greedy_matches_reference_expressions():
    f = load("config1_greedy.npz")
    bonus, accept, eos = OAc.greedy_posterior(f["draft"], f["target_logits"], int(f["eos"]))
    np.testing.assert_array_equal(bonus, f["bonus"])
    np.testing.assert_array_equal(accept, f["accept"])
    np.testing.assert_array_equal(eos, f["eos_accepted"])


def test_chain_matches_float64_sequential_rule():
    f = load("chain_small.npz")
    ids, acc, emi = OAc.chain_probs(f["draft_probs"], f["draft"], f["target_probs"], f["uniforms"])
    np.testing.assert_array_equal(ids, f["ids"])
    np.testing.assert_array_equal(acc, f["accepted"])
    np.testing.assert_array_equal(emi, f["emitted"])
    assert 0 < f["emitted"].mean() < 3  # both accept and reject branches occur
