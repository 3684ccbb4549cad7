"""Randomized acceptance cases, each checked bit for bit against the CPU oracle: the
stochastic chain over logits (mtp_engine.py:561-575), the greedy evaluation under both
accept rules (mtp_engine.py:553-560), and the softmax of get_sampling_probs
(batchspec/backends/utils/sampling.py:18-58).  The cases mix the three logit dtypes,
vocabularies with a partial last group (V % 8 != 0) and below one group per lane, draft
lengths 0-7, temperatures, scales, integer-valued (tied) logits, -inf padding, a peaked
token, and one-hot drafts."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import sampling as S
from oracle import accept as OAc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
N_CASES = 60


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _case(rng):
    dt = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
    V = int(rng.choice([2, 7, 64, 1001, 4096, 32000, 128256, 151936]))
    B = int(rng.integers(1, 40 if V <= 32000 else 10))
    k = int(rng.integers(0, 8))
    T = float(rng.choice([0.3, 0.7, 1.0, 2.0]))
    sigma = float(rng.choice([0.05, 1.0, 3.0, 8.0]))
    kind = str(rng.choice(["plain", "quant", "pad", "peak"]))
    onehot = bool(rng.random() < 0.3)
    return dt, V, B, k, T, sigma, kind, onehot, int(rng.integers(1 << 30))


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_acceptance_case(case):
    dt, V, B, k, T, sigma, kind, onehot, seed = _case(np.random.default_rng(1000 + case))
    say(f"case {case}: {dt} B={B} k={k} V={V} T={T} sigma={sigma} kind={kind} onehot={onehot}")
    g = torch.Generator().manual_seed(seed)
    t = torch.randn((B, k + 1, V), generator=g) * sigma
    d = t[:, :k] + torch.randn((B, k, V), generator=g) * 0.5
    if kind == "quant":
        t, d = torch.round(t), torch.round(d)
    elif kind == "pad" and V > 8:
        t[..., -(V // 5):] = -float("inf")
        d[..., -(V // 5):] = -float("inf")
    elif kind == "peak":
        t[..., V // 2] += 15.0
        d[..., V // 2] += 15.0
    t, d = t.to(DT[dt]), d.to(DT[dt])
    am = t[:, :k].float().argmax(-1)
    ids = torch.where(torch.rand((B, k), generator=g) < 0.6, am,
                      torch.randint(0, V, (B, k), generator=g))
    u = torch.rand((B, k + 1), generator=g)

    ref = OAc.chain_logits(None if onehot else d.float().numpy(), ids.numpy(),
                           t.float().numpy(), T, u.numpy())
    got = S.chain_speculative_sampling_from_logits(None if onehot else d.to(DEV), ids.to(DEV),
                                                   t.to(DEV), T, uniforms=u.to(DEV))
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r, err_msg="chain")

    for rule in ["reference", "prefix"]:
        gb, ga, ge = bsx.evaluate_posterior(ids.to(DEV), t.to(DEV), greedy=True,
                                            eos_token_id=int(V // 3), accept_rule=rule)
        rb, ra, re_ = OAc.greedy_posterior(ids.numpy(), t.float().numpy(), int(V // 3), rule=rule)
        np.testing.assert_array_equal(gb.cpu().numpy(), rb, err_msg=f"greedy {rule}")
        np.testing.assert_array_equal(ga.cpu().numpy(), ra, err_msg=f"greedy {rule}")
        np.testing.assert_array_equal(ge.cpu().numpy(), re_, err_msg=f"greedy {rule}")

    sp = S.softmax(t.to(DEV), temperature=T)
    sref = OAc.softmax(t.float().reshape(-1, V).numpy(), T).reshape(sp.shape)
    np.testing.assert_array_equal(sp.cpu().numpy().view(np.int32),
                                  sref.astype(np.float32).view(np.int32), err_msg="softmax")
