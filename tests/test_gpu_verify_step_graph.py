"""A whole speculative verify step captured in one graph and replayed while the batch's
lengths change: DevicePageTable.insert_kv (batchspec/backends/base/page_table.py:55-93),
the fused KV append (kv_cache.py:47-84), plan(on_device=True) and run()
(attn_wrapper.py:33-72, standard.py:69), logits from the attention output, the greedy
evaluate_posterior (mtp_engine.py:553-560) and delete_kv of the rejected tokens
(page_table.py:95-137).  Every replay is compared with the same step run eagerly on a
copy of the state: page table, cache, attention output and accept counts bit for bit;
the first step's attention also against the fp32 oracle."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd.page import append_kv
from batchspec_amd.page_table import DevicePageTable
from oracle import attention as OA

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


B, K, H, HKV, D, PS, MAXP, V = 8, 4, 32, 8, 128, 16, 40, 8
S = K + 1


class State:
    def __init__(self, seed):
        g = torch.Generator().manual_seed(seed)
        self.pt = DevicePageTable(PS, B, MAXP, DEV)
        self.cache = torch.zeros((B * MAXP, 2, PS, HKV, D), dtype=torch.bfloat16, device=DEV)
        ctx = torch.randint(40, 300, (B,), generator=g)
        self.pt.insert_kv(ctx.to(DEV))
        indptr = torch.cat([torch.zeros(1, dtype=torch.int64), ctx.cumsum(0)]).to(torch.int32)
        k = (torch.randn((int(ctx.sum()), HKV, D), generator=g) * 0.5).to(torch.bfloat16).to(DEV)
        v = (torch.randn((int(ctx.sum()), HKV, D), generator=g) * 0.5).to(torch.bfloat16).to(DEV)
        append_kv(k, v, indptr.to(DEV), self.cache, self.pt.paged_kv_indptr,
                  self.pt.paged_kv_indices, self.pt.paged_kv_last_page_len)
        self.ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)

    def clone(self):
        c = State.__new__(State)
        c.pt = DevicePageTable(PS, B, MAXP, DEV)
        for name in ("cachelens", "paged_kv_indptr", "paged_kv_indices", "paged_kv_last_page_len"):
            getattr(c.pt, name).copy_(getattr(self.pt, name))
        c.pt.page_manager.num_allocated_pages.copy_(self.pt.page_manager.num_allocated_pages)
        c.cache = self.cache.clone()
        c.ws = torch.empty_like(self.ws)
        return c


class Inputs:
    """The step's inputs, in buffers a graph captures."""

    def __init__(self, w_proj):
        self.q = torch.zeros((B * S, H, D), dtype=torch.bfloat16, device=DEV)
        self.k = torch.zeros((B * S, HKV, D), dtype=torch.bfloat16, device=DEV)
        self.v = torch.zeros_like(self.k)
        self.draft = torch.zeros((B, K), dtype=torch.int64, device=DEV)
        self.out = torch.zeros_like(self.q)
        self.accept = torch.zeros(B, dtype=torch.int64, device=DEV)
        self.qo_indptr = (torch.arange(B + 1, dtype=torch.int32) * S).to(DEV)
        self.w_proj = w_proj

    def fill(self, seed):
        g = torch.Generator().manual_seed(seed)
        self.q.copy_((torch.randn(self.q.shape, generator=g) * 0.5).to(torch.bfloat16))
        self.k.copy_((torch.randn(self.k.shape, generator=g) * 0.5).to(torch.bfloat16))
        self.v.copy_((torch.randn(self.v.shape, generator=g) * 0.5).to(torch.bfloat16))
        self.draft.copy_(torch.randint(0, V, (B, K), generator=g))


def verify_step(st, x, wrapper):
    st.pt.insert_kv(S)
    append_kv(x.k, x.v, x.qo_indptr, st.cache, st.pt.paged_kv_indptr, st.pt.paged_kv_indices,
              st.pt.paged_kv_last_page_len)
    wrapper.plan(x.qo_indptr, st.pt.paged_kv_indptr, st.pt.paged_kv_indices,
                 st.pt.paged_kv_last_page_len, H, HKV, D, PS, causal=True,
                 q_data_type=torch.bfloat16, on_device=True, max_qo_len=S)
    wrapper.run(x.q, st.cache, out=x.out)
    logits = (x.out.float().reshape(B * S, H * D) @ x.w_proj).reshape(B, S, V)
    _, acc, _ = bsx.evaluate_posterior(x.draft, logits, greedy=True, eos_token_id=-1)
    x.accept.copy_(acc)
    st.pt.delete_kv(S - acc)


def test_verify_step_graph_replays_with_changing_lengths():
    say("verify step in one graph: insert, append, device plan, attention, greedy accept, delete")
    w_proj = (torch.randn((H * D, V), generator=torch.Generator().manual_seed(3)) * 0.05).to(DEV)
    st_g = State(11)
    st_e = st_g.clone()
    xg, xe = Inputs(w_proj), Inputs(w_proj)
    wg = bsx.BatchPrefillWithPagedKVCacheWrapper(st_g.ws, "NHD", use_cuda_graph=True,
                                                 paged_kv_indices_buf=st_g.pt.paged_kv_indices)
    we = bsx.BatchPrefillWithPagedKVCacheWrapper(st_e.ws, "NHD")

    # one warm-up step on both states (outside the graph), then capture the step on
    # the graph's state (capturing executes nothing)
    xg.fill(100)
    xe.fill(100)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        verify_step(st_g, xg, wg)  # warm-up: a real step on the graph's state
    torch.cuda.current_stream().wait_stream(side)
    verify_step(st_e, xe, we)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        verify_step(st_g, xg, wg)
    torch.cuda.synchronize()

    lens_seen = set()
    for step in range(4):
        xg.fill(200 + step)
        xe.fill(200 + step)
        if step == 0:
            pre = st_e.clone()
        graph.replay()
        verify_step(st_e, xe, we)
        torch.cuda.synchronize()
        for name in ("cachelens", "paged_kv_indptr", "paged_kv_last_page_len"):
            assert torch.equal(getattr(st_g.pt, name), getattr(st_e.pt, name)), (step, name)
        n = int(st_e.pt.paged_kv_indptr[-1])
        assert torch.equal(st_g.pt.paged_kv_indices[:n], st_e.pt.paged_kv_indices[:n])
        assert torch.equal(st_g.cache, st_e.cache), step
        assert torch.equal(xg.out, xe.out), step
        assert torch.equal(xg.accept, xe.accept), step
        lens_seen.add(tuple(st_e.pt.cachelens.cpu().tolist()))
        if step == 0:
            # the step's attention against the oracle, on the state after insert + append
            cl = pre.pt.cachelens.cpu().numpy() + S
            pages = (cl + PS - 1) // PS
            kvp = np.concatenate([[0], np.cumsum(pages)])
            idx = np.concatenate([np.arange(b * MAXP, b * MAXP + pages[b]) for b in range(B)])
            last = (cl - 1) % PS + 1
            ref = OA.verify_attention(xe.q.float().cpu().numpy(), st_e.cache.float().cpu().numpy(),
                                      xe.qo_indptr.cpu().numpy(), kvp, idx, last, PS,
                                      mode="causal")
            err = np.abs(xe.out.float().cpu().numpy() - ref) - (2e-2 + 2e-2 * np.abs(ref))
            assert err.max() <= 0
        assert st_g.pt.errors.item() == 0 and wg.device_plan_error() == 0
    assert len(lens_seen) == 4  # the lengths changed at every step
