"""GPU parity of the KV append and of acceptance (through the C ABI) against the oracle.
Bar: bit-exact (appended pages, argmax, accepted lengths and token ids, and — for the
shared canonical order — the softmax probabilities themselves)."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import sampling as S
from batchspec_amd.workloads import config2, greedy_case, make_verify_batch, stochastic_case
from oracle import accept as OAc
from oracle import append as OAp

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _bits(t):
    return t.view(torch.int16).cpu().numpy() if t.element_size() == 2 else t.cpu().numpy().view(np.int32)


# ---------------------------------------------------------------- append
def _append_case(b):
    nnz = b.k_new.shape[0]
    ref = OAp.update(_bits(b.k_new).reshape(nnz, b.num_kv_heads, -1),
                     _bits(b.v_new).reshape(nnz, b.num_kv_heads, -1),
                     b.qo_indptr.cpu().numpy(), _bits(b.cache), b.kv_indptr.cpu().numpy(),
                     b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(), b.page_size)
    return ref


@pytest.mark.parametrize("ps,dtype", [(16, torch.bfloat16), (1, torch.bfloat16), (8, torch.float16),
                                      (32, torch.float32)])
def test_fused_append_bit_exact(ps, dtype):
    say(f"fused append ps={ps} {dtype}")
    b = make_verify_batch(7, 0, 300, 5, 32, 8, 128, ps, dtype=dtype, seed=ps, extra_pages=5,
                          qo_lens=np.array([5, 1, 0, 9, 5, 2, 5])).to(DEV)
    ref = _append_case(b)
    cache = bsx.StandardKVCache(b.cache.shape[0], ps, 8, 128, dtype=dtype, device=DEV)
    cache.kv_cache.copy_(b.cache)

    class PT:
        paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len = (
            b.kv_indptr, b.kv_indices, b.kv_last_page_len)

    out = cache.update(b.k_new, b.v_new, b.qo_indptr, PT)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(out), ref)


def test_split_append_api_bit_exact():
    say("get_seq_lens / get_batch_indices_positions / append_paged_kv_cache")
    b = make_verify_batch(9, 10, 500, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=9).to(DEV)
    ref = _append_case(b)
    sl = bsx.get_seq_lens(b.kv_indptr, b.kv_last_page_len, 16)
    np.testing.assert_array_equal(sl.cpu().numpy(), b.kv_lens)
    nnz = b.k_new.shape[0]
    bi, pos = bsx.get_batch_indices_positions(b.qo_indptr, sl, nnz)
    rbi, rpos = OAp.get_batch_indices_positions(b.qo_indptr.cpu().numpy(), b.kv_lens, nnz)
    np.testing.assert_array_equal(bi.cpu().numpy(), rbi)
    np.testing.assert_array_equal(pos.cpu().numpy(), rpos)
    cache = b.cache.clone()
    bsx.append_paged_kv_cache(b.k_new, b.v_new, bi, pos, cache, b.kv_indices, b.kv_indptr,
                              b.kv_last_page_len, "NHD")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(cache), ref)


def test_config2_append_bit_exact():
    say("config 2 append (320 tokens x 8 heads)")
    b = config2(device=DEV)
    ref = _append_case(b)
    cache = b.cache.clone()
    bsx.append_kv(b.k_new, b.v_new, b.qo_indptr, cache, b.kv_indptr, b.kv_indices,
                  b.kv_last_page_len)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(cache), ref)


# ---------------------------------------------------------------- argmax / greedy
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("V", [7, 1000, 128256])
def test_argmax_bit_exact(dtype, V):
    say(f"argmax {dtype} V={V}")
    g = torch.Generator().manual_seed(V)
    x = torch.randn((37, V), generator=g).to(dtype)
    x[3, :] = 0.0
    x[4, 5 % V] = float("nan")
    x[4, 2 % V] = float("nan")
    x[5, :] = -float("inf")
    x[6, :] = x[6, 0]
    x[7, V // 2] = 1e4
    x[7, V - 1] = 1e4
    x[8, :] = -0.0
    x[8, V - 1] = 0.0
    got = S.argmax(x.to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, OAc.argmax(x.float().numpy()))
    np.testing.assert_array_equal(got, x.float().argmax(-1).numpy())


@pytest.mark.parametrize("rule", ["reference", "prefix"])
def test_greedy_posterior_ids_and_logits(rule):
    say(f"greedy evaluate_posterior rule={rule}")
    for V, dtype in [(1000, torch.float32), (128256, torch.bfloat16)]:
        c = greedy_case(B=64, k=4, V=V, seed=V, dtype=dtype)
        eos = int(c.draft_tokens[0, 1])
        ref = OAc.greedy_posterior(c.draft_tokens.numpy(), c.target_logits.float().numpy(), eos,
                                   rule)
        for preds in (c.target_logits.to(DEV), torch.from_numpy(OAc.argmax(
                c.target_logits.float().numpy())).to(DEV)):
            bonus, acc, eos_acc = bsx.evaluate_posterior(c.draft_tokens.to(DEV), preds, greedy=True,
                                                         eos_token_id=eos, accept_rule=rule)
            assert bonus.shape == (64, 1) and bonus.dtype == torch.int64
            assert acc.shape == (64,) and acc.dtype == torch.int64
            assert eos_acc.shape == (64, 1) and eos_acc.dtype == torch.bool
            np.testing.assert_array_equal(bonus.cpu().numpy(), ref[0])
            np.testing.assert_array_equal(acc.cpu().numpy(), ref[1])
            np.testing.assert_array_equal(eos_acc.cpu().numpy(), ref[2])


def test_greedy_logits_repeated_calls_and_shapes():
    """Back-to-back calls reusing one cached workspace across shapes agree with the
    oracle (row counts from 6 to 3000, one to many parts per row)."""
    say("greedy repeated calls / large batch")
    for B, k, V in [(64, 4, 128256), (3, 1, 50), (600, 4, 1000)]:
        c = greedy_case(B=B, k=k, V=V, seed=B + V, dtype=torch.bfloat16)
        eos = int(c.draft_tokens[0, 0])
        ref = OAc.greedy_posterior(c.draft_tokens.numpy(), c.target_logits.float().numpy(), eos,
                                   "reference")
        logits, draft = c.target_logits.to(DEV), c.draft_tokens.to(DEV)
        for i in range(6):
            bonus, acc, eos_acc = bsx.evaluate_posterior(draft, logits, greedy=True,
                                                         eos_token_id=eos)
            np.testing.assert_array_equal(bonus.cpu().numpy(), ref[0], err_msg=f"B={B} call {i}")
            np.testing.assert_array_equal(acc.cpu().numpy(), ref[1], err_msg=f"B={B} call {i}")
            np.testing.assert_array_equal(eos_acc.cpu().numpy(), ref[2], err_msg=f"B={B} call {i}")


# ---------------------------------------------------------------- softmax / chain
@pytest.mark.parametrize("dtype,V,T", [(torch.float32, 1000, 1.0), (torch.bfloat16, 128256, 1.0),
                                       (torch.bfloat16, 32000, 0.6), (torch.float16, 4099, 1.3)])
def test_softmax_bit_exact(dtype, V, T):
    say(f"softmax {dtype} V={V} T={T}")
    g = torch.Generator().manual_seed(V)
    x = (torch.randn((12, V), generator=g) * 3).to(dtype)
    x[1, 17] = -float("inf")
    got = S.softmax(x.to(DEV), T).cpu().numpy()
    ref = OAc.softmax(x.float().numpy(), T)
    np.testing.assert_array_equal(got.view(np.int32), ref.view(np.int32))


def test_softmax_edge_rows_bit_exact():
    # rows whose lanes start at -inf, rows that raise every lane's maximum at every group
    # (ascending), large logits inside the domain (|x*C| < 2^31) and beyond it (Z NaN in
    # both; NaN payloads are not compared)
    V = 128256
    say(f"softmax edge rows bf16 V={V}")
    g = torch.Generator().manual_seed(11)
    x = torch.randn((6, V), generator=g) * 2
    x[0, : 8 * 2048 * 3] = -float("inf")
    x[1] = torch.sort(x[1]).values
    x[2] = torch.sort(x[2], descending=True).values
    x[3] = x[3] * 1e6
    x[4] = x[4] * 1e8
    x[5] = x[5] * 1e10
    x = x.to(torch.bfloat16)
    got = S.softmax(x.to(DEV), 1.0).cpu().numpy()
    ref = OAc.softmax(x.float().numpy(), 1.0)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(got[fin].view(np.int32), ref[fin].view(np.int32))
    assert np.all(np.isfinite(got[:5]))
    assert np.isnan(got[5]).all()


@pytest.mark.parametrize("onehot", [False, True])
@pytest.mark.parametrize("V", [1000, 32000])
def test_chain_probs_bit_exact(onehot, V):
    say(f"chain probs V={V} onehot={onehot}")
    rng = np.random.default_rng(V + onehot)
    B, k = 48, 5
    tl = rng.normal(0, 2, size=(B, k + 1, V)).astype(np.float32)
    p = OAc.softmax(tl)
    q = None if onehot else OAc.softmax(tl[:, :k] + rng.normal(0, 0.7, size=(B, k, V)).astype(np.float32))
    ids = rng.integers(0, V, size=(B, k))
    u = rng.random((B, k + 1)).astype(np.float32)
    ref = OAc.chain_probs(q, ids, p, u)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    got = S.chain_speculative_sampling(t(q), t(ids), t(p), uniforms=t(u))
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)


@pytest.mark.parametrize("onehot,T", [(False, 1.0), (True, 1.0), (False, 0.7)])
def test_chain_logits_bit_exact_small(onehot, T):
    say(f"chain logits small onehot={onehot} T={T}")
    c = stochastic_case(B=32, k=4, V=3000, temperature=T, seed=17)
    ref = OAc.chain_logits(None if onehot else c.draft_logits.float().numpy(),
                           c.draft_tokens.numpy(), c.target_logits.float().numpy(), T,
                           c.uniforms.numpy())
    got = S.chain_speculative_sampling_from_logits(None if onehot else c.draft_logits.to(DEV),
                                                   c.draft_tokens.to(DEV),
                                                   c.target_logits.to(DEV), T,
                                                   uniforms=c.uniforms.to(DEV))
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)


@pytest.mark.parametrize("V", [3000, 128256])
def test_chain_logits_no_residual_mass_draws_from_target(V):
    # draft rows equal to the target rows and every draft token at a -inf logit of both:
    # p(x) = q(x) = 0 rejects position 0, the residual max(0, p - q) has no mass, and the
    # emitted token is drawn from p_0 itself (the pick kernel's second tree)
    B, k = 6, 3
    say(f"chain logits without residual mass V={V}")
    g = torch.Generator().manual_seed(V + 5)
    tl = (torch.randn((B, k + 1, V), generator=g) * 2).to(torch.bfloat16)
    ids = torch.randint(0, V, (B, k), generator=g)
    for b in range(B):
        for i in range(k):
            tl[b, i, ids[b, i]] = -float("inf")
    dl = tl[:, :k].clone()
    u = torch.rand((B, k + 1), generator=g)
    ref = OAc.chain_logits(dl.float().numpy(), ids.numpy(), tl.float().numpy(), 1.0, u.numpy())
    got = S.chain_speculative_sampling_from_logits(dl.to(DEV), ids.to(DEV), tl.to(DEV), 1.0,
                                                   uniforms=u.to(DEV))
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)
    out = got[0].cpu().numpy()
    assert (got[2].cpu().numpy() == 0).all()  # every request stops at position 0
    for b in range(B):
        assert 0 <= out[b, 0] < V and np.isfinite(tl[b, 0, out[b, 0]].float().item())


def test_config5_full_size_bit_exact():
    say("config 5 full size: B=128, k=5, V=128256, bf16, T=1")
    c = stochastic_case(device=DEV)
    got = S.chain_speculative_sampling_from_logits(c.draft_logits, c.draft_tokens,
                                                   c.target_logits, 1.0, uniforms=c.uniforms)
    ref = OAc.chain_logits(c.draft_logits.float().cpu().numpy(), c.draft_tokens.cpu().numpy(),
                           c.target_logits.float().cpu().numpy(), 1.0, c.uniforms.cpu().numpy())
    for a, r in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), r)
    emitted = got[2].cpu().numpy()
    assert 0 < emitted.mean() < 5  # both rejections and full acceptances occur


def test_evaluate_posterior_sampling_branch():
    say("evaluate_posterior sampling branch (one-hot draft, T=0.8)")
    c = stochastic_case(B=16, k=4, V=5000, temperature=0.8, seed=23)
    bonus, acc, eos = bsx.evaluate_posterior(c.draft_tokens.to(DEV), c.target_logits.to(DEV),
                                             greedy=False, eos_token_id=7, temperature=0.8,
                                             uniforms=c.uniforms.to(DEV))
    out, _, emi = OAc.chain_logits(None, c.draft_tokens.numpy(), c.target_logits.float().numpy(),
                                   0.8, c.uniforms.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), emi + 1)
    np.testing.assert_array_equal(bonus[:, 0].cpu().numpy(), out[np.arange(16), emi])
    np.testing.assert_array_equal(eos[:, 0].cpu().numpy(), (out == 7).any(1))


def test_greedy_graph_keeps_its_workspace_after_a_larger_call():
    """A graph captured at a small batch replays into the workspace it captured, even
    after an eager call at a larger batch has grown the cached workspace: the outgrown
    buffer is kept, so no tensor allocated afterwards shares its memory."""
    say("greedy: capture at B=16, eager at B=64, then replay")
    from batchspec_amd import posterior
    posterior._WS.clear()
    small = greedy_case(B=16, k=4, V=128256, seed=16, dtype=torch.bfloat16)
    big = greedy_case(B=64, k=4, V=128256, seed=64, dtype=torch.bfloat16)
    ds, ls = small.draft_tokens.to(DEV), small.target_logits.to(DEV)
    ref = OAc.greedy_posterior(small.draft_tokens.numpy(), small.target_logits.float().numpy(),
                               -1, "reference")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        bsx.evaluate_posterior(ds, ls, greedy=True, eos_token_id=-1)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = bsx.evaluate_posterior(ds, ls, greedy=True, eos_token_id=-1)
    bsx.evaluate_posterior(big.draft_tokens.to(DEV), big.target_logits.to(DEV), greedy=True,
                           eos_token_id=-1)
    nbytes = posterior._WS["__retired__"][-1].numel()
    probes = [torch.full((nbytes // 4,), 12345, dtype=torch.int32, device=DEV) for _ in range(4)]
    torch.cuda.synchronize()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(outs[0].cpu().numpy(), ref[0], err_msg=f"replay {rep}")
        np.testing.assert_array_equal(outs[1].cpu().numpy(), ref[1], err_msg=f"replay {rep}")
        for p in probes:
            assert bool((p == 12345).all()), f"replay {rep} wrote into a live tensor"
