"""The stochastic chain acceptance over logits (batchspec/backends/mtp_engine.py:561-575),
unfiltered and with the top-k / top-p filters of get_sampling_probs
(batchspec/backends/utils/sampling.py:50-56), captured in one graph and replayed on new
logits, draft tokens and uniforms written into the captured buffers.  Each replay is
compared bit for bit with the same call run eagerly on copies, with eager work and
synchronisations between the replays; the first replay also against the CPU oracle.  The
settings reach every filter kernel: listed rows, rows finished by the deferred kernel
(top-p alone, top_k above 64) and whole-row draws from tile sums."""
import sys

import numpy as np
import pytest
import torch

from batchspec_amd import sampling as S
from oracle import accept as OAc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
B, K, V = 8, 4, 32000


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _fill(tl, dl, ids, u, seed, sigma):
    """Target N(0, sigma), draft = target + N(0, 0.5); draft tokens the draft argmax with
    probability 0.7, else uniform; uniforms U(0, 1)."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn((B, K + 1, V), generator=g) * sigma
    d = t[:, :K] + torch.randn((B, K, V), generator=g) * 0.5
    am = d.argmax(-1)
    rnd = torch.randint(0, V, (B, K), generator=g)
    keep = torch.rand((B, K), generator=g) < 0.7
    tl.copy_(t.to(torch.bfloat16))
    dl.copy_(d.to(torch.bfloat16))
    ids.copy_(torch.where(keep, am, rnd))
    u.copy_(torch.rand((B, K + 1), generator=g))


@pytest.mark.parametrize("top_k,top_p", [(0, 1.0), (20, 0.95), (0, 0.95), (2000, 0.0)])
def test_chain_sampling_graph_replays(top_k, top_p):
    say(f"chain sampling in a graph: B={B} k={K} V={V} top_k={top_k} top_p={top_p}")
    tl = torch.zeros((B, K + 1, V), dtype=torch.bfloat16, device=DEV)
    dl = torch.zeros((B, K, V), dtype=torch.bfloat16, device=DEV)
    ids = torch.zeros((B, K), dtype=torch.int64, device=DEV)
    u = torch.zeros((B, K + 1), dtype=torch.float32, device=DEV)
    _fill(tl, dl, ids, u, seed=0, sigma=2.0)

    def step():
        return S.chain_speculative_sampling_from_logits(dl, ids, tl, 1.0, uniforms=u,
                                                        top_k=top_k, top_p=top_p)

    step()  # allocates the workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    torch.cuda.synchronize()
    for rep, sigma in enumerate([2.0, 0.3, 6.0, 2.0, 1.0]):
        _fill(tl, dl, ids, u, seed=100 + rep, sigma=sigma)
        ref = S.chain_speculative_sampling_from_logits(dl.clone(), ids.clone(), tl.clone(), 1.0,
                                                       uniforms=u.clone(), top_k=top_k,
                                                       top_p=top_p)
        ref = [r.cpu().numpy() for r in ref]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.cpu().numpy() for o in out]
        for a, r in zip(got, ref):
            np.testing.assert_array_equal(a, r, err_msg=f"replay {rep} sigma={sigma}")
        if rep == 0:
            want = OAc.chain_filtered(dl.float().cpu().numpy(), ids.cpu().numpy(),
                                      tl.float().cpu().numpy(), 1.0, top_k, top_p,
                                      u.cpu().numpy())
            for a, r in zip(got, want):
                np.testing.assert_array_equal(a, r, err_msg="replay 0 against the oracle")


@pytest.mark.parametrize("top_k,top_p", [(20, 0.95), (0, 0.95), (2000, 0.0), (0, 1.0)])
def test_sample_and_sampling_probs_graph_replays(top_k, top_p):
    """sample() and get_sampling_probs (batchspec/backends/utils/sampling.py:18-115) captured
    in one graph, replayed on new logits and uniforms written into the captured buffers;
    each replay equals the same calls run eagerly on copies, the first also the oracle."""
    R, Sq, V2 = 16, 1, 32000
    say(f"sample + sampling probs in a graph: rows={R} V={V2} top_k={top_k} top_p={top_p}")
    lg = torch.zeros((R, Sq, V2), dtype=torch.bfloat16, device=DEV)
    uu = torch.zeros((R, Sq), dtype=torch.float32, device=DEV)

    def fill(seed, sigma):
        g = torch.Generator().manual_seed(seed)
        lg.copy_((torch.randn((R, Sq, V2), generator=g) * sigma).to(torch.bfloat16))
        uu.copy_(torch.rand((R, Sq), generator=g))

    def step():
        ids = S.sample(lg, top_p, top_k, 0.8, uniforms=uu)
        probs = S.get_sampling_probs(lg, top_p, top_k, 0.8)
        return ids, probs

    fill(0, 2.0)
    step()  # allocates the workspaces outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    torch.cuda.synchronize()
    for rep, sigma in enumerate([2.0, 0.3, 6.0, 2.0]):
        fill(200 + rep, sigma)
        ref_ids = S.sample(lg.clone(), top_p, top_k, 0.8, uniforms=uu.clone()).cpu().numpy()
        ref_p = S.get_sampling_probs(lg.clone(), top_p, top_k, 0.8).cpu().numpy()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out[0].cpu().numpy(), ref_ids, err_msg=f"ids, replay {rep}")
        np.testing.assert_array_equal(out[1].cpu().numpy().view(np.int32), ref_p.view(np.int32),
                                      err_msg=f"probs, replay {rep}")
        if rep == 0:
            x = lg.float().cpu().numpy().reshape(R * Sq, V2)
            want = OAc.filtered_probs(x, 0.8, top_k, top_p)
            np.testing.assert_array_equal(out[1].cpu().numpy().reshape(R * Sq, V2).view(np.int32),
                                          want.view(np.int32), err_msg="probs against the oracle")
            want_ids = OAc.sample(x, 0.8, top_k, top_p, uu.cpu().numpy().reshape(-1))
            np.testing.assert_array_equal(out[0].cpu().numpy().reshape(-1), want_ids,
                                          err_msg="ids against the oracle")
