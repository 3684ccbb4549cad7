"""gfx950 kernels (through the C ABI) against the committed golden fixtures."""
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import sampling

pytestmark = pytest.mark.gpu
G = Path(__file__).resolve().parent / "golden"
DEV = "cuda:0"


def load(name):
    return dict(np.load(G / name, allow_pickle=False))


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def t(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return x if dtype is None else x.to(dtype)


def test_attention_bf16_vs_float64_sdpa():
    """Config-1 inputs rounded to bf16 against the fp32-input float64 SDPA output:
    |gpu - ref| <= 2e-2 + 2e-2 |ref|."""
    say("golden: config-1 attention")
    f = load("config1_attention.npz")
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(t(f["qo_indptr"]), t(f["kv_indptr"]), t(f["kv_indices"]), t(f["kv_last_page_len"]),
           8, 2, 64, int(f["page_size"]), causal=True, q_data_type=torch.bfloat16)
    out, lse = w.run(t(f["q"], torch.bfloat16), t(f["cache"], torch.bfloat16), return_lse=True)
    g = out.float().cpu().numpy()
    err = np.abs(g - f["out"]) - (2e-2 + 2e-2 * np.abs(f["out"]))
    assert err.max() <= 0, np.abs(g - f["out"]).max()
    np.testing.assert_allclose(lse.cpu().numpy(), f["lse"], atol=5e-2, rtol=1e-2)


def test_append_bit_exact_slots():
    say("golden: config-1 append")
    a = load("config1_attention.npz")
    f = load("config1_append.npz")
    cache = t(a["cache"])
    before = cache.clone()
    bsx.append_kv(t(f["k_new"]), t(f["v_new"]), t(a["qo_indptr"]), cache, t(a["kv_indptr"]),
                  t(a["kv_indices"]), t(a["kv_last_page_len"]))
    torch.cuda.synchronize()
    c = cache.cpu().numpy()
    P, S = f["target_page"], f["target_slot"]
    np.testing.assert_array_equal(c[P, 0, S], f["k_new"])
    np.testing.assert_array_equal(c[P, 1, S], f["v_new"])
    touched = np.zeros(c.shape[:3], bool)
    touched[P, :, S] = True
    np.testing.assert_array_equal(c[~touched], before.cpu().numpy()[~touched])


def test_greedy_posterior_bit_exact():
    say("golden: config-1 greedy acceptance")
    f = load("config1_greedy.npz")
    bonus, accept, eos = bsx.evaluate_posterior(t(f["draft"]), t(f["target_logits"]), greedy=True,
                                                eos_token_id=int(f["eos"]))
    np.testing.assert_array_equal(bonus.cpu().numpy(), f["bonus"])
    np.testing.assert_array_equal(accept.cpu().numpy(), f["accept"])
    np.testing.assert_array_equal(eos.cpu().numpy(), f["eos_accepted"])


def test_chain_speculative_sampling_bit_exact():
    say("golden: chain speculative sampling, V=16")
    f = load("chain_small.npz")
    ids, acc, emi = sampling.chain_speculative_sampling(
        t(f["draft_probs"]), t(f["draft"]), t(f["target_probs"]), uniforms=t(f["uniforms"]))
    np.testing.assert_array_equal(ids.cpu().numpy(), f["ids"])
    np.testing.assert_array_equal(acc.cpu().numpy(), f["accepted"])
    np.testing.assert_array_equal(emi.cpu().numpy(), f["emitted"])
