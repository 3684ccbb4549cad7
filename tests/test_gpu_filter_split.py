"""The few-rows path of the top-k filter (filter_parts_kernel + filter_combine_kernel:
each row over four workgroups by quarters of its canonical lanes, then one combine per
row), taken for top_k <= 64 with at most 512 rows of 16384..262144 logits, bit-exact
against the oracle (oracle/filter.c): the reference's default sampling acceptance at the
MTP verify shape (64 x 5 rows of 128256, T=0.6, top_k=20, top_p=0.95, one-hot drafts,
mtp_engine.py:561-575), get_sampling_probs and sample() on that path, and the cases that
send a row to the exact threshold search (ties filling a part's list, -inf padding, a
first round without k finite maxima), plus fp32 rows with a partial last group."""
import sys

import numpy as np
import pytest
import torch

from batchspec_amd import sampling as S
from batchspec_amd.workloads import greedy_case
from oracle import accept as OAc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_default_sampling_acceptance_at_the_mtp_shape():
    """[64, 5, 128256] bf16 target logits, one-hot drafts (target argmax with probability
    0.7), T=0.6, top_k=20, top_p=0.95: the bench's sampling_accept_mtp workload."""
    say("split rows: default sampling acceptance, [64, 5, 128256] bf16")
    g = greedy_case(B=64, k=4, V=128256, p_match=0.7, seed=2002, dtype=torch.bfloat16)
    got = S.chain_speculative_sampling_from_logits(None, g.draft_tokens.to(DEV),
                                                   g.target_logits.to(DEV), 0.6,
                                                   uniforms=g.uniforms.to(DEV), top_k=20,
                                                   top_p=0.95)
    ref = OAc.chain_filtered(None, g.draft_tokens.numpy(), g.target_logits.float().numpy(), 0.6,
                             20, 0.95, g.uniforms.numpy())
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)
    say(f"  accepted {int(got[2].sum()) + 64} tokens")


def _rows(n, V, dtype, seed, sigma=2.0, quantize=None, pad_inf=0, flat_first=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((n, V), generator=g) * sigma
    if quantize:
        x = torch.round(x * quantize) / quantize
    if pad_inf:
        x[:, V - pad_inf:] = -float("inf")
    if flat_first:
        # the first 16384 logits -inf except a handful: some parts' first rounds hold fewer
        # than k finite maxima
        x[:, :16384] = -float("inf")
        x[:, 100:105] = 3.0
    return x.to(dtype)


@pytest.mark.parametrize("dt,V,top_k,top_p,kw", [
    (torch.bfloat16, 32768, 20, 0.95, dict(quantize=1.0)),      # ties: parts cannot list
    (torch.bfloat16, 65536, 20, 0.0, dict(pad_inf=30000)),      # -inf tail
    (torch.float16, 40000, 64, 0.9, dict(flat_first=True)),     # first rounds mostly -inf
    (torch.float32, 20004, 20, 0.95, {}),                       # partial last group (fp32)
    (torch.bfloat16, 262144, 1, 0.0, {}),                       # top-1, largest split vocab
    (torch.bfloat16, 128256, 64, 0.5, dict(sigma=0.3)),          # flat rows, top-p cuts first
])
def test_split_rows_probs_and_samples(dt, V, top_k, top_p, kw):
    say(f"split rows: get_sampling_probs and sample(), {dt} V={V} top_k={top_k} top_p={top_p} {kw}")
    x = _rows(24, V, dt, seed=V + top_k, **kw)
    T = 0.8
    got = S.get_sampling_probs(x.to(DEV), top_p=top_p, top_k=top_k, temperature=T)
    ref = OAc.filtered_probs(x.float().numpy(), T, top_k, top_p)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(ref.shape).view(np.int32),
                                  ref.view(np.int32))
    u = torch.rand(24, generator=torch.Generator().manual_seed(V))
    ids = S.sample(x.to(DEV), top_p=top_p, top_k=top_k, temperature=T, uniforms=u.to(DEV))
    np.testing.assert_array_equal(ids.cpu().numpy().reshape(-1),
                                  OAc.sample(x.float().numpy(), T, top_k, top_p, u.numpy()))


def test_split_rows_with_draft_logits_and_many_rows():
    """B=40, k=5 with draft logits: 440 rows (the split path's bound is 512)."""
    say("split rows: chain with draft logits, B=40 k=5 V=32000")
    g = torch.Generator().manual_seed(9)
    t = torch.randn((40, 6, 32000), generator=g) * 2
    d = t[:, :5] + torch.randn((40, 5, 32000), generator=g) * 0.5
    t, d = t.to(torch.bfloat16), d.to(torch.bfloat16)
    rng = np.random.default_rng(9)
    ids = OAc.sample(d.float().reshape(-1, 32000).numpy(), 1.0, 20, 0.95,
                     rng.random(200, dtype=np.float32)).reshape(40, 5)
    u = rng.random((40, 6), dtype=np.float32)
    ids_t = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int64))
    got = S.chain_speculative_sampling_from_logits(d.to(DEV), ids_t.to(DEV), t.to(DEV), 1.0,
                                                   uniforms=torch.from_numpy(u).to(DEV), top_k=20,
                                                   top_p=0.95)
    ref = OAc.chain_filtered(d.float().numpy(), ids, t.float().numpy(), 1.0, 20, 0.95, u)
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)


@pytest.mark.parametrize("k,top_k,top_p,sigma,quantize", [
    (4, 20, 0.95, 2.0, 1.0),   # ties: parts that cannot list, requests on the fallback
    (1, 20, 0.95, 2.0, None),
    (3, 24, 0.0, 2.0, None),   # the largest top_k of the one-launch tail, top-k alone
    (7, 5, 0.5, 8.0, None),    # eight rows (two per wave); peaked rows: the nucleus cuts first
    (8, 20, 0.95, 2.0, None),  # nine rows: the combine and chain kernels instead
    (2, 1, 0.0, 0.05, 64.0),   # top-1 with ties at the maximum
])
def test_one_hot_chain_on_the_request_kernel(k, top_k, top_p, sigma, quantize):
    """One-hot drafts over split rows (the combine and the chain of each request in one
    workgroup for k + 1 <= 8 and top_k <= 24), with draft ids out of range in some
    requests, bit-exact against the oracle."""
    say(f"split rows, one-hot chain: k={k} top_k={top_k} top_p={top_p} sigma={sigma} q={quantize}")
    B, V = 12, 32000
    x = _rows(B * (k + 1), V, torch.bfloat16, seed=100 + k, sigma=sigma, quantize=quantize)
    t = x.reshape(B, k + 1, V)
    rng = np.random.default_rng(k)
    am = t.float().argmax(-1)[:, :k].numpy()
    ids = np.where(rng.random((B, k)) < 0.7, am, rng.integers(0, V, (B, k))).astype(np.int64)
    if k:
        ids[1, 0] = -1
        ids[2, k - 1] = V
    u = rng.random((B, k + 1), dtype=np.float32)
    got = S.chain_speculative_sampling_from_logits(None, torch.from_numpy(ids).to(DEV), t.to(DEV),
                                                   0.6, uniforms=torch.from_numpy(u).to(DEV),
                                                   top_k=top_k, top_p=top_p)
    ref = OAc.chain_filtered(None, ids, t.float().numpy(), 0.6, top_k, top_p, u)
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)
