"""The wrapper built and driven exactly as BatchSpec's MTP engine drives FlashInfer's.

Construction follows batchspec/backends/base/attn_wrapper.py:53-70 with the buffers of
batchspec/backends/mtp_engine.py:120-140: ``use_cuda_graph=True``, a fixed
``qo_indptr_buf`` of max_batch + 1 entries, the page table's three ``paged_kv_*``
buffers, and the MTP ``custom_mask_buf`` (max_batch * (k+1)^2 * max_cache_len / 8 + 1
bytes) and ``mask_indptr_buf``.  Each step then does what
MTPEngine.pre_draft_and_verify does (mtp_engine.py:399-432): insert (k+1)^2 tokens,
build the bool mask cat(ones(S, cachelen_b), common_mask) per request, and plan with
qo_indptr * S, causal=False, custom_mask=mask.  run() is captured once; later steps
re-plan with other cache lengths and replay the graph, which must equal an eager run of
the same plan bit for bit and the fp32 oracle within the north-star tolerance."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import masks as M
from batchspec_amd.page import append_kv
from batchspec_amd.page_table import DevicePageTable
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
MAXB, K, HQ, HKV, D, PS, MAX_LEN = 6, 4, 32, 8, 128, 16, 1200
S = (K + 1) ** 2
MAX_CACHE = MAX_LEN + S + 1
MAXP = (MAX_CACHE + PS - 1) // PS + 2


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class Engine:
    """The buffers of MTPEngine.setup_caches and the wrapper of _create_attention_wrapper."""

    def __init__(self):
        self.pt = DevicePageTable(PS, MAXB, MAXP, DEV)
        self.cache = (torch.randn((MAXB * MAXP, 2, PS, HKV, D), generator=torch.Generator(
            device=DEV).manual_seed(5), device=DEV) * 0.5).to(torch.bfloat16)
        self.qo_indptr = torch.arange(MAXB + 1, dtype=torch.int32, device=DEV)
        self.attn_buffer = torch.empty(384 << 20, dtype=torch.uint8, device=DEV)
        self.custom_mask_buf = torch.empty(MAXB * S * MAX_CACHE // 8 + 1, dtype=torch.uint8,
                                           device=DEV)
        self.mask_indptr_buf = torch.arange(MAXB + 1, dtype=torch.int32, device=DEV)
        self.wrapper = bsx.BatchPrefillWithPagedKVCacheWrapper(
            float_workspace_buffer=self.attn_buffer, kv_layout="NHD", use_cuda_graph=True,
            qo_indptr_buf=self.qo_indptr, paged_kv_indptr_buf=self.pt.paged_kv_indptr,
            paged_kv_indices_buf=self.pt.paged_kv_indices,
            paged_kv_last_page_len_buf=self.pt.paged_kv_last_page_len,
            custom_mask_buf=self.custom_mask_buf, mask_indptr_buf=self.mask_indptr_buf)

    def pre_draft_and_verify(self):
        cachelens = self.pt.cachelens.cpu().tolist()
        mask = M.mtp_verify_custom_mask(cachelens, K, device=DEV)
        self.pt.insert_kv(S)
        self.wrapper.plan(qo_indptr=self.qo_indptr * S, paged_kv_indptr=self.pt.paged_kv_indptr,
                          paged_kv_indices=self.pt.paged_kv_indices,
                          paged_kv_last_page_len=self.pt.paged_kv_last_page_len,
                          num_qo_heads=HQ, num_kv_heads=HKV, head_dim_qk=D, page_size=PS,
                          q_data_type=torch.bfloat16, causal=False, custom_mask=mask)
        return cachelens, mask


def _oracle(e, q, mask):
    """fp32 oracle on the wrapper's current page table with the engine's bool mask."""
    from oracle import attention as OA
    kvp = e.pt.paged_kv_indptr.cpu().numpy()
    n = int(kvp[-1])
    return OA.verify_attention(q.float().cpu().numpy(), e.cache.float().cpu().numpy(),
                               (np.arange(MAXB + 1) * S).astype(np.int32), kvp,
                               e.pt.paged_kv_indices[:n].cpu().numpy(),
                               e.pt.paged_kv_last_page_len.cpu().numpy(), PS, mode="custom",
                               custom_mask=mask.cpu().numpy(), return_lse=True)


def test_mtp_engine_construction_plan_capture_replan_replay():
    say("wrapper built as attn_wrapper.py:53-70, MTP custom mask, capture then re-plan")
    e = Engine()
    g = torch.Generator().manual_seed(1)
    e.pt.insert_kv(torch.randint(200, MAX_LEN - 3 * S, (MAXB,), generator=g).to(DEV))
    q = torch.empty((MAXB * S, HQ, D), dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(q)
    lse = torch.empty((MAXB * S, HQ), dtype=torch.float32, device=DEV)
    graph = None
    for step in range(3):
        cachelens, mask = e.pre_draft_and_verify()
        q.copy_((torch.randn(q.shape, generator=g) * 0.5).to(torch.bfloat16))
        # this step's draft tokens get fresh K/V, as the layer's append would write
        kv = (torch.randn((MAXB * S, HKV, D), generator=g) * 0.5).to(torch.bfloat16).to(DEV)
        append_kv(kv, kv.flip(0).contiguous(), e.qo_indptr * S, e.cache, e.pt.paged_kv_indptr,
                  e.pt.paged_kv_indices, e.pt.paged_kv_last_page_len)
        plan = e.wrapper.plan_info
        assert plan.mask_mode == 2 and plan.device_plan == 1
        eager_o, eager_l = e.wrapper.run(q, e.cache, return_lse=True)
        eager_o, eager_l = eager_o.clone(), eager_l.clone()
        if graph is None:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                e.wrapper.run(q, e.cache, out=out, lse=lse)
            torch.cuda.current_stream().wait_stream(s)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                e.wrapper.run(q, e.cache, out=out, lse=lse)
        for rep in range(2):
            out.zero_()
            lse.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager_o), f"step {step} replay {rep}"
            assert torch.equal(lse, eager_l), f"step {step} replay {rep} lse"
        ref_o, ref_l = _oracle(e, q, mask)
        err, mx = AP.check(out, ref_o, lse, ref_l)
        say(f"  step {step}: cachelens {cachelens}, max err {err:.3g} (max|ref| {mx:.3g})")
        # accept a few tokens per request and drop the rest, as after verification
        acc = torch.randint(1, K + 2, (MAXB,), generator=g)
        e.pt.delete_kv((S - acc).to(torch.int32).to(DEV))
    # the mask words live in the engine's custom_mask_buf
    assert e.wrapper._mask_words.data_ptr() == e.custom_mask_buf.data_ptr()


def _chain_mask(kv_lens, qo_lens):
    """Flattened per-request bool masks: every prefix column visible, a causal block over
    the last qo_len columns (the layout plan(custom_mask=...) accepts)."""
    parts = []
    for L, n in zip(kv_lens, qo_lens):
        if n == 0:
            continue
        parts.append(torch.cat((torch.ones((n, L - n), dtype=torch.bool),
                                torch.tril(torch.ones((n, n), dtype=torch.bool))), 1).flatten())
    return torch.cat(parts).to(DEV)


def _plan_custom(e, qo_lens):
    """plan() with the engine's page table, causal=False and a bool custom mask for the
    given query tokens per request (the MTP engine's call, mtp_engine.py:420-432)."""
    qo = torch.from_numpy(np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)).to(DEV)
    kvp = e.pt.paged_kv_indptr.cpu().numpy().astype(np.int64)
    last = e.pt.paged_kv_last_page_len.cpu().numpy().astype(np.int64)
    kv_lens = [int((kvp[b + 1] - kvp[b] - 1) * PS + last[b]) for b in range(MAXB)]
    e.wrapper.plan(qo, e.pt.paged_kv_indptr, e.pt.paged_kv_indices, e.pt.paged_kv_last_page_len,
                   HQ, HKV, D, PS, q_data_type=torch.bfloat16, causal=False,
                   custom_mask=_chain_mask(kv_lens, qo_lens))
    return qo


def _capture(e, q, out, lse=None):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        e.wrapper.run(q, e.cache, out=out, lse=lse)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        e.wrapper.run(q, e.cache, out=out, lse=lse)
    return graph


def test_replan_beyond_the_captured_shape_is_refused():
    """Same custom-mask plan arguments; only the query tokens per request grow (S + 1
    against the captured S), so the refusal comes from the shape alone.  A plan that
    fits the captured shape afterwards is accepted and its replay equals an eager run."""
    say("graph mode: a plan needing a larger shape after a capture raises")
    e = Engine()
    e.pt.insert_kv(300)
    e.pt.insert_kv(S + 1)
    _plan_custom(e, [S] * MAXB)
    q = torch.zeros((MAXB * S, HQ, D), dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(q)
    graph = _capture(e, q, out)
    # the same shape with other lengths is accepted
    e.pt.insert_kv(7)
    _plan_custom(e, [S] * MAXB)
    # S + 1 query tokens per request exceed the captured S; mask and heads unchanged
    with pytest.raises(ValueError, match="captured"):
        _plan_custom(e, [S + 1] * MAXB)
    # the refused plan left the captured shape in place: a fitting plan still replays
    e.pt.insert_kv(3)
    _plan_custom(e, [S] * MAXB)
    q.copy_((torch.randn(q.shape, generator=torch.Generator().manual_seed(3)) * 0.5)
            .to(torch.bfloat16))
    out.zero_()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    eager = e.wrapper.run(q, e.cache)
    torch.cuda.synchronize()
    assert torch.equal(out, eager)


def test_replan_with_more_query_tokens_than_the_captured_buffers_is_refused():
    """The captured run() read q and wrote out / lse of (MAXB - 2) * S rows (two idle
    requests with no query tokens).  A later plan of the same fixed shape with every
    request live has MAXB * S query tokens: replaying it would run past those buffers,
    so plan() refuses it."""
    say("graph mode: a plan with more query tokens than the captured q / out holds raises")
    e = Engine()
    e.pt.insert_kv(400)
    e.pt.insert_kv(S)
    live = [S] * (MAXB - 2) + [0, 0]
    _plan_custom(e, live)
    rows = (MAXB - 2) * S
    q = torch.zeros((rows, HQ, D), dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(q)
    lse = torch.empty((rows, HQ), dtype=torch.float32, device=DEV)
    _capture(e, q, out, lse)
    _plan_custom(e, live)  # the captured total is accepted again
    with pytest.raises(ValueError, match="token rows"):
        _plan_custom(e, [S] * MAXB)
    torch.cuda.synchronize()


def test_plan_refuses_a_table_past_the_page_ids():
    say("plan: paged_kv_indptr[-1] beyond paged_kv_indices is refused")
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    qo = torch.tensor([0, 5, 10], dtype=torch.int32, device=DEV)
    kvp = torch.tensor([0, 3, 9], dtype=torch.int32, device=DEV)
    last = torch.tensor([16, 4], dtype=torch.int32, device=DEV)
    idx = torch.arange(8, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="exceeds"):
        w.plan(qo, kvp, idx, last, 32, 8, 128, 16, causal=True, q_data_type=torch.bfloat16)
    w.plan(qo, kvp, idx, last, 32, 8, 128, 16, causal=True, q_data_type=torch.bfloat16,
           on_device=True, max_qo_len=5)
    sentinel = torch.full((10, 32, 128), 7.0, dtype=torch.bfloat16, device=DEV)
    w.run(torch.zeros_like(sentinel), torch.zeros((9, 2, 16, 8, 128), dtype=torch.bfloat16,
                                                  device=DEV), out=sentinel)
    torch.cuda.synchronize()
    assert w.device_plan_error() == -1
    assert (sentinel == 7.0).all()
