"""GPU parity of the top-k / top-p filter (batchspec/backends/utils/sampling.py:50-56)
fused into acceptance (mtp_engine.py:561-575), get_sampling_probs and sample()
(sampling.py:61-115), through the C ABI, against the CPU oracle (oracle/filter.c).
Bar: bit-exact (token ids, accept counts, and the fp32 filtered probabilities).
Cases cover the listed fast path, the radix fallback (ties, top_k above the list
capacity, a nucleus wider than the bound), rows that are not 16-byte multiples, and
the three logit types."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import sampling as S
from batchspec_amd.workloads import stochastic_case
from oracle import accept as OAc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _case(B, k, V, dtype, T, top_k, top_p, seed, sigma=2.0, quantize=None, draft_from="filtered"):
    """Target N(0, sigma), draft = target + N(0, 0.5); draft tokens drawn by the oracle from
    the filtered draft distribution (or the target argmax for an MTP-like one-hot case)."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn((B, k + 1, V), generator=g) * sigma
    d = t[:, :k] + torch.randn((B, k, V), generator=g) * 0.5
    if quantize:
        t = torch.round(t * quantize) / quantize
        d = torch.round(d * quantize) / quantize
    t = t.to(dtype)
    d = d.to(dtype)
    rng = np.random.default_rng(seed)
    if draft_from == "filtered" and k > 0:
        ids = OAc.sample(d.float().reshape(-1, V).numpy(), T, top_k, top_p,
                         rng.random(B * k, dtype=np.float32)).reshape(B, k)
    else:
        am = t[:, :k].float().argmax(-1).numpy()
        ids = np.where(rng.random((B, k)) < 0.7, am, rng.integers(0, V, (B, k)))
    u = rng.random((B, k + 1), dtype=np.float32)
    return t, d, torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int64)), torch.from_numpy(u)


CHAIN_CASES = [
    # dtype, onehot, B, k, V, T, top_k, top_p, quantize
    ("bf16", True, 8, 4, 32000, 0.6, 20, 0.95, None),      # reference defaults, MTP draft
    ("bf16", False, 8, 4, 32000, 1.0, 20, 0.95, None),
    ("fp16", False, 6, 3, 20000, 0.8, 50, 0.0, None),      # top-k alone
    ("fp32", True, 6, 3, 20000, 1.0, 0, 0.9, None),        # top-p alone (fallback for flat rows)
    ("bf16", False, 4, 3, 12000, 1.0, 20, 0.95, 2.0),      # heavy ties -> radix select
    ("bf16", True, 4, 2, 8000, 1.0, 300, 0.0, None),       # top_k above the list capacity
    ("fp16", False, 5, 3, 1003, 0.7, 10, 0.8, None),       # ragged rows (V % 8 != 0)
    ("fp32", False, 5, 2, 777, 1.0, 1, 0.0, None),         # top-1
    ("bf16", False, 6, 3, 5000, 1.2, 4000, 0.999, None),   # nucleus wider than the list
]


@pytest.mark.parametrize("dt,onehot,B,k,V,T,top_k,top_p,q", CHAIN_CASES)
def test_filtered_chain_bit_exact(dt, onehot, B, k, V, T, top_k, top_p, q):
    say(f"filtered chain {dt} onehot={onehot} B={B} k={k} V={V} T={T} top_k={top_k} "
        f"top_p={top_p} quantize={q}")
    t, d, ids, u = _case(B, k, V, DT[dt], T, top_k, top_p, seed=V + 7 * top_k + len(dt),
                         quantize=q, draft_from="argmax" if onehot else "filtered")
    ref = OAc.chain_filtered(None if onehot else d.float().numpy(), ids.numpy(),
                             t.float().numpy(), T, top_k, top_p, u.numpy())
    got = S.chain_speculative_sampling_from_logits(None if onehot else d.to(DEV), ids.to(DEV),
                                                   t.to(DEV), T, uniforms=u.to(DEV),
                                                   top_k=top_k, top_p=top_p)
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)


@pytest.mark.parametrize("dt,V,T,top_k,top_p,q", [
    ("bf16", 32000, 0.6, 20, 0.95, None),
    ("fp16", 5001, 1.0, 0, 0.7, None),
    ("fp32", 4096, 0.9, 100, 0.0, None),
    ("bf16", 6000, 1.0, 20, 0.9, 2.0),
    ("bf16", 3000, 1.0, 0, 0.99, None),
])
def test_sampling_probs_bit_exact(dt, V, T, top_k, top_p, q):
    say(f"get_sampling_probs {dt} V={V} T={T} top_k={top_k} top_p={top_p} quantize={q}")
    t, _, _, _ = _case(3, 3, V, DT[dt], T, top_k, top_p, seed=V % 97, quantize=q,
                       draft_from="argmax")
    got = S.get_sampling_probs(t.to(DEV), top_p=top_p, top_k=top_k, temperature=T)
    ref = OAc.filtered_probs(t.float().reshape(-1, V).numpy(), T, top_k, top_p).reshape(t.shape)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.int32), ref.view(np.int32))


@pytest.mark.parametrize("dt,V,T,top_k,top_p", [
    ("bf16", 128256, 1.0, 0, 0.95),     # wide nucleus: about a third of the row
    ("bf16", 128256, 1.0, 0, 0.5),
    ("bf16", 128256, 1.0, 2000, 0.9),   # top_k above the list capacity
    ("fp16", 128256, 0.7, 5000, 0.0),
    ("fp32", 50000, 1.5, 0, 0.99),
    ("bf16", 40000, 0.3, 0, 0.999),     # low temperature: thresholds far down the exponent axis
])
def test_sampling_probs_large_thresholds(dt, V, T, top_k, top_p):
    """Upper sets too large to list: the threshold comes from the exponent-bin
    histogram and a walk of one bin."""
    say(f"get_sampling_probs, large threshold: {dt} V={V} T={T} top_k={top_k} top_p={top_p}")
    g = torch.Generator().manual_seed(V + top_k)
    x = (torch.randn((3, V), generator=g) * 2).to(DT[dt])
    got = S.get_sampling_probs(x.to(DEV), top_p=top_p, top_k=top_k, temperature=T)
    ref = OAc.filtered_probs(x.float().numpy(), T, top_k, top_p)
    np.testing.assert_array_equal(got.cpu().numpy().reshape(ref.shape).view(np.int32),
                                  ref.view(np.int32))


def _band_rows(rows, V, n_band, lo, width, seed):
    """fp32 N(0, 2) rows with n_band elements of each replaced by values spread over
    [lo, lo + width): many elements inside one bin of the weight's exponent."""
    g = np.random.default_rng(seed)
    x = (g.standard_normal((rows, V)) * 2).astype(np.float32)
    for r in range(rows):
        idx = g.choice(V, n_band, replace=False)
        x[r, idx] = (lo + width * g.random(n_band)).astype(np.float32)
    return x


@pytest.mark.parametrize("n_band,by", [(20000, "top_k"), (20000, "top_p"), (600, "top_k"),
                                       (600, "top_p"), (3000, "top_p")])
def test_sampling_probs_dense_bin(n_band, by):
    """The threshold inside a narrow band of many values: a bin of more than 1024
    elements (a second histogram over its sub-bins) or of a few hundred (narrowed in
    LDS).  The cut is placed in the middle of the band."""
    say(f"get_sampling_probs, dense bin: band of {n_band}, cut by {by}")
    V, lo, width, T = 60000, 2.0, 0.01, 1.0
    x = _band_rows(2, V, n_band, lo, width, seed=n_band)
    mid = lo + width / 2
    if by == "top_k":
        top_k, top_p = int((x[0] >= mid).sum()), 0.0
    else:
        w = np.exp((x[0].astype(np.float64) - x[0].max()) / T)
        top_k, top_p = 0, float(w[x[0] >= mid].sum() / w.sum())
    got = S.get_sampling_probs(torch.from_numpy(x).to(DEV), top_p=top_p, top_k=top_k,
                               temperature=T)
    ref = OAc.filtered_probs(x, T, top_k, top_p)
    kept = (ref[0] > 0).sum()
    assert abs(int(kept) - int((x[0] >= mid).sum())) < n_band // 4  # the cut is in the band
    np.testing.assert_array_equal(got.cpu().numpy().reshape(ref.shape).view(np.int32),
                                  ref.view(np.int32))


@pytest.mark.parametrize("dt,V,T,top_k,top_p", [
    ("bf16", 32000, 0.6, 20, 0.95), ("fp16", 999, 1.0, 0, 0.5), ("fp32", 2048, 1.0, 0, 1.0),
    ("bf16", 5000, 0.8, 700, 0.0),
    ("bf16", 128256, 1.0, 0, 0.95),   # whole-row draws from tile sums, no draft
])
def test_sample_bit_exact(dt, V, T, top_k, top_p):
    say(f"sample {dt} V={V} T={T} top_k={top_k} top_p={top_p}")
    g = torch.Generator().manual_seed(V)
    x = (torch.randn((4, 16, V), generator=g) * 2).to(DT[dt])
    u = torch.rand(64, generator=g)
    got = S.sample(x.to(DEV), top_p=top_p, top_k=top_k, temperature=T, uniforms=u.to(DEV))
    assert got.dtype == torch.int64 and got.shape == (4, 16)
    ref = OAc.sample(x.float().reshape(-1, V).numpy(), T, top_k, top_p, u.numpy())
    np.testing.assert_array_equal(got.reshape(-1).cpu().numpy(), ref)


def test_evaluate_posterior_filtered():
    say("evaluate_posterior sampling branch with top_k=20, top_p=0.95, T=0.6")
    t, _, ids, u = _case(16, 4, 20000, torch.bfloat16, 0.6, 20, 0.95, seed=31, draft_from="argmax")
    bonus, acc, eos = bsx.evaluate_posterior(ids.to(DEV), t.to(DEV), greedy=False,
                                             eos_token_id=7, temperature=0.6, top_p=0.95,
                                             top_k=20, uniforms=u.to(DEV))
    out, _, emi = OAc.chain_filtered(None, ids.numpy(), t.float().numpy(), 0.6, 20, 0.95,
                                     u.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), emi + 1)
    np.testing.assert_array_equal(bonus[:, 0].cpu().numpy(), out[np.arange(16), emi])
    np.testing.assert_array_equal(eos[:, 0].cpu().numpy(), (out == 7).any(1))


@pytest.mark.parametrize("top_k,top_p", [(20, 0.95), (0, 0.95), (2000, 0.0)])
def test_config5_shape_filtered_subset(top_k, top_p):
    say(f"config-5 row shape (V=128256, k=5) with top_k={top_k}, top_p={top_p}: 24 requests")
    c = stochastic_case(B=24, k=5, seed=1005)
    got = S.chain_speculative_sampling_from_logits(c.draft_logits.to(DEV), c.draft_tokens.to(DEV),
                                                   c.target_logits.to(DEV), 1.0,
                                                   uniforms=c.uniforms.to(DEV), top_k=top_k,
                                                   top_p=top_p)
    ref = OAc.chain_filtered(c.draft_logits.float().numpy(), c.draft_tokens.numpy(),
                             c.target_logits.float().numpy(), 1.0, top_k, top_p,
                             c.uniforms.numpy())
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)


def test_repeated_calls_reuse_workspace():
    say("filtered chain: three calls of different shapes on one workspace")
    for B, k, V, tk, tp in [(8, 4, 20000, 20, 0.95), (3, 1, 500, 0, 0.6), (8, 4, 20000, 5, 0.0)]:
        t, d, ids, u = _case(B, k, V, torch.bfloat16, 1.0, tk, tp, seed=B * V + tk)
        ref = OAc.chain_filtered(d.float().numpy(), ids.numpy(), t.float().numpy(), 1.0, tk, tp,
                                 u.numpy())
        got = S.chain_speculative_sampling_from_logits(d.to(DEV), ids.to(DEV), t.to(DEV), 1.0,
                                                       uniforms=u.to(DEV), top_k=tk, top_p=tp)
        for a, r in zip(got, ref):
            np.testing.assert_array_equal(a.cpu().numpy(), r)


def test_randomized_filtered_chains():
    """40 random cases (dtype, one-hot or draft logits, B, k, V, T, top_k, top_p, value
    scale, quantisation for ties), bit-exact against the oracle."""
    say("filtered chain: 40 randomized cases")
    rng = np.random.default_rng(2024)
    for case in range(40):
        dt = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
        onehot = bool(rng.random() < 0.4)
        B = int(rng.integers(1, 7))
        k = int(rng.integers(0, 5))
        V = int(rng.choice([17, 255, 1000, 4099, 9000, 20000]))
        T = float(rng.choice([0.3, 0.6, 1.0, 1.7]))
        top_k = int(rng.choice([0, 1, 3, 20, 64, 300, V - 1, V + 5]))
        top_p = float(rng.choice([0.0, 0.3, 0.8, 0.95, 0.999, 1.0]))
        sigma = float(rng.choice([0.2, 2.0, 6.0]))
        q = None if rng.random() < 0.7 else float(rng.choice([1.0, 4.0]))
        t, d, ids, u = _case(B, k, V, DT[dt], T, top_k, top_p, seed=int(rng.integers(1 << 30)),
                             sigma=sigma, quantize=q, draft_from="argmax" if onehot else "filtered")
        ref = OAc.chain_filtered(None if onehot else d.float().numpy(), ids.numpy(),
                                 t.float().numpy(), T, top_k, top_p, u.numpy())
        got = S.chain_speculative_sampling_from_logits(None if onehot else d.to(DEV), ids.to(DEV),
                                                       t.to(DEV), T, uniforms=u.to(DEV),
                                                       top_k=top_k, top_p=top_p)
        for a, r in zip(got, ref):
            np.testing.assert_array_equal(a.cpu().numpy(), r, err_msg=f"case {case}: {dt} onehot="
                                          f"{onehot} B={B} k={k} V={V} T={T} top_k={top_k} "
                                          f"top_p={top_p} sigma={sigma} q={q}")


def test_randomized_large_thresholds():
    """30 random rows sets on the paths for upper sets too large to list (top-p alone,
    top_k above 64): N(0, sigma) rows, some with -inf padding, ties from quantisation or a
    dense band of values, ragged lengths and the three logit types; the filtered
    probabilities bit-exact against the oracle."""
    say("get_sampling_probs: 30 randomized large-threshold cases")
    rng = np.random.default_rng(77)
    for case in range(30):
        dt = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
        V = int(rng.choice([1500, 4099, 20000, 65537]))
        T = float(rng.choice([0.5, 1.0, 2.0]))
        if rng.random() < 0.5:
            top_k, top_p = 0, float(rng.choice([0.3, 0.9, 0.99, 0.9999]))
        else:
            top_k = int(rng.choice([65, 300, 1500, V // 2]))
            top_p = float(rng.choice([0.0, 0.9, 0.99]))
        sigma = float(rng.choice([0.5, 2.0, 6.0]))
        x = rng.standard_normal((2, V)) * sigma
        kind = rng.choice(["plain", "quantized", "band", "padded"])
        if kind == "quantized":
            x = np.round(x * 4) / 4
        elif kind == "band":
            idx = rng.choice(V, V // 4, replace=False)
            x[:, idx] = 1.0 + 0.01 * rng.random((2, V // 4))
        elif kind == "padded":
            x[:, -(V // 10):] = -np.inf
        xt = torch.from_numpy(x.astype(np.float32)).to(DT[dt])
        got = S.get_sampling_probs(xt.to(DEV), top_p=top_p, top_k=top_k, temperature=T)
        ref = OAc.filtered_probs(xt.float().numpy(), T, top_k, top_p)
        np.testing.assert_array_equal(
            got.cpu().numpy().reshape(ref.shape).view(np.int32), ref.view(np.int32),
            err_msg=f"case {case}: {dt} V={V} T={T} top_k={top_k} top_p={top_p} sigma={sigma} "
                    f"kind={kind}")


def test_randomized_filter_mix():
    """200 random cases over every filter setting class (top_k 0/1/small/at and above 64,
    1024, 1025, V-1, V; top_p 0 .. 1), temperatures 0.2-3, one-hot and logit drafts,
    vocabularies 17-128256 and five row shapes: plain N(0, sigma), quantised (ties), a
    dense band, -inf padding, one dominant token.  Chain outputs and the filtered
    probabilities bit-exact against the oracle."""
    say("filtered chain + get_sampling_probs: 200 randomized mixed cases")
    rng = np.random.default_rng(606)
    for case in range(200):
        dt = ["bf16", "fp16", "fp32"][int(rng.integers(3))]
        onehot = bool(rng.random() < 0.3)
        B, k = int(rng.integers(1, 6)), int(rng.integers(0, 5))
        V = int(rng.choice([17, 300, 1025, 4099, 20000, 50001, 128256]))
        T = float(rng.choice([0.2, 0.7, 1.0, 1.5, 3.0]))
        top_k = int(rng.choice([0, 1, 5, 20, 64, 65, 200, 1024, 1025, 3000, V - 1, V]))
        top_p = float(rng.choice([0.0, 0.1, 0.5, 0.9, 0.95, 0.999, 1.0]))
        sigma = float(rng.choice([0.1, 1.0, 2.0, 5.0]))
        kind = str(rng.choice(["plain", "quant", "band", "pad", "peak"]))
        g = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
        t = torch.randn((B, k + 1, V), generator=g) * sigma
        d = t[:, :k] + torch.randn((B, k, V), generator=g) * 0.5
        if kind == "quant":
            t, d = torch.round(t * 2) / 2, torch.round(d * 2) / 2
        elif kind == "band" and V > 100:
            idx = torch.randperm(V, generator=g)[:V // 5]
            t[..., idx] = 1.0 + 0.01 * torch.rand((B, k + 1, V // 5), generator=g)
        elif kind == "pad" and V > 20:
            t[..., -(V // 7):] = -float("inf")
            d[..., -(V // 7):] = -float("inf")
        elif kind == "peak":
            t[..., 0] += 12.0
            d[..., 0] += 12.0
        t, d = t.to(DT[dt]), d.to(DT[dt])
        ids = torch.randint(0, V, (B, k), generator=g)
        u = torch.rand((B, k + 1), generator=g)
        msg = (f"case {case}: {dt} onehot={onehot} B={B} k={k} V={V} T={T} top_k={top_k} "
               f"top_p={top_p} sigma={sigma} kind={kind}")
        ref = OAc.chain_filtered(None if onehot else d.float().numpy(), ids.numpy(),
                                 t.float().numpy(), T, top_k, top_p, u.numpy())
        got = S.chain_speculative_sampling_from_logits(None if onehot else d.to(DEV), ids.to(DEV),
                                                       t.to(DEV), T, uniforms=u.to(DEV),
                                                       top_k=top_k, top_p=top_p)
        for a, r in zip(got, ref):
            np.testing.assert_array_equal(a.cpu().numpy(), r, err_msg=msg)
        pr = S.get_sampling_probs(t.to(DEV), top_p=top_p, top_k=top_k, temperature=T)
        pref = OAc.filtered_probs(t.float().reshape(-1, V).numpy(), T, top_k, top_p)
        np.testing.assert_array_equal(pr.cpu().numpy().reshape(pref.shape).view(np.int32),
                                      pref.view(np.int32), err_msg=msg)
