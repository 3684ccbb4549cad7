"""GPU tests of the device-side attention schedule (bsx_attn_plan_device through
plan(on_device=True)): the blob equals the CPU restatement (oracle/attn_schedule.py)
entry for entry, attention run on it matches the fp32 oracle under the checks of
tests/attn_parity.py (the north star's elementwise 2e-2 plus the normalised bounds and
the lse), with planted keys and guards at the benchmark shapes so a dropped mask, a
lost last tile or an all-zeros output fails; a graph holding plan and run replays
correctly after the page table changes, and a malformed table yields the error code
and an empty schedule."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd.workloads import config2, make_verify_batch
from oracle import attention as OA
from oracle import attn_schedule as OS
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check(got, ref, lse_got=None, lse_ref=None):
    """The full-size check of tests/attn_parity.py: elementwise 2e-2 + 2e-2|ref|, max
    error within 2e-2 max|ref|, relative L2 within 1e-2, lse within 5e-3."""
    return AP.check(got, ref, lse_got, lse_ref)


def oracle(b, mode, **kw):
    return OA.verify_attention(b.q.float().cpu().numpy(), b.cache.float().cpu().numpy(),
                               b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                               b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(),
                               b.page_size, mode=mode, return_lse=True, **kw)


def wrapper(mb=256, **kw):
    return bsx.BatchPrefillWithPagedKVCacheWrapper(
        torch.empty(mb << 20, dtype=torch.uint8, device=DEV), "NHD", **kw)


def device_plan(w, b, max_qo, causal=True, **kw):
    w.plan(b.qo_indptr.to(DEV), b.kv_indptr.to(DEV), b.kv_indices.to(DEV),
           b.kv_last_page_len.to(DEV), b.num_qo_heads, b.num_kv_heads, b.head_dim, b.page_size,
           causal=causal, q_data_type=b.q.dtype, on_device=True, max_qo_len=max_qo, **kw)


def blob_of(w):
    p = w.plan_info
    torch.cuda.synchronize()
    return OS.read_blob(w._ws[: p.plan_ints * 4].view(torch.int32).cpu().numpy(), p.batch,
                        p.num_ctas)


def compare_schedule(w, b, max_qo, mode=1, sink=0, window=0):
    p = w.plan_info
    got = blob_of(w)
    want = OS.schedule(b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                       b.kv_last_page_len.cpu().numpy(), b.page_size, mode, sink, window, max_qo,
                       p.num_ctas)
    for k in want:
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)
    OS.check_invariants(got, b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                        b.kv_last_page_len.cpu().numpy(), b.page_size, mode, sink, window)
    return got


def run_lse(w, b):
    out, lse = w.run(b.q, b.cache, return_lse=True)
    torch.cuda.synchronize()
    return out, lse


def planted_check_with_guards(w, b, seed, progress=0):
    """Plant keys at the device plan's segment boundaries, tile boundaries and the draft
    block, run again on the same plan, compare with the per-request oracle (output and
    lse), and show the check rejects zeros, a dropped causal mask and a dropped last tile
    on these very inputs."""
    segs = blob_of(w)["segments"]
    AP.plant_keys(b, "causal", segments=segs, seed=seed)
    out, lse = run_lse(w, b)
    res = AP.oracle_per_request(b, "causal", mutations=("nomask", "droplast"), progress=progress)
    e, m = check(out, res[None][0], lse, res[None][1])
    say(f"  planted: max err {e:.3g} (max|ref| {m:.3g}), {len(segs)} segments, "
        f"{int(blob_of(w)['dyn'][0])} split requests")
    AP.assert_discriminates(res[None], [("zeros", np.zeros_like(res[None][0]), None),
                                        ("no mask", *res["nomask"]),
                                        ("last tile dropped", *res["droplast"])])


def test_config2_on_device_plan():
    """Config 2 (B=64, ctx 1k-4k, 5 causal queries, 32/8 heads, D=128) on the device
    plan the one-graph verify step uses: plain inputs, then planted keys with guards."""
    say("device plan, config 2: plain inputs")
    b = config2(device=DEV)
    w = wrapper()
    device_plan(w, b, 5)
    out, lse = run_lse(w, b)
    compare_schedule(w, b, 5)
    assert w.device_plan_error() == 0
    ref = AP.oracle_per_request(b, "causal")[None]
    e, m = check(out, ref[0], lse, ref[1])
    say(f"  plain: max err {e:.3g} (max|ref| {m:.3g})")
    say("device plan, config 2: planted keys")
    planted_check_with_guards(w, b, seed=12)


def test_long_contexts_on_device_plan():
    """B=32, ctx 20k-40k on the device plan (every request split and merged through the
    bound-sized partial slots), against the per-request fp32 oracle with planted keys
    at the plan's segment boundaries; guards: zeros, no mask, dropped last tile."""
    say("device plan, B=32 ctx 20k-40k: planted keys")
    b = make_verify_batch(32, 20000, 40000, 5, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=37, device=DEV)
    w = wrapper()
    device_plan(w, b, 5)
    compare_schedule(w, b, 5)
    assert w.device_plan_error() == 0
    assert int(blob_of(w)["dyn"][0]) == 32, "every request should be split at this size"
    planted_check_with_guards(w, b, seed=13, progress=8)


@pytest.mark.parametrize("B,lo,hi,qo,hq,hkv,d", [(7, 10, 300, 3, 28, 4, 128),
                                                 (200, 1, 600, 1, 8, 2, 64)])
def test_small_causal_chains_on_device_plan(B, lo, hi, qo, hq, hkv, d):
    say(f"device plan, causal chain: B={B} ctx=[{lo},{hi}] qo={qo} H={hq}/{hkv} D={d}")
    b = make_verify_batch(B, lo, hi, qo, hq, hkv, d, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=B + qo).to(DEV)
    w = wrapper()
    device_plan(w, b, qo)
    out, lse = run_lse(w, b)
    compare_schedule(w, b, qo)
    ref, ref_lse = oracle(b, "causal")
    check(out, ref, lse, ref_lse)
    assert w.device_plan_error() == 0


def test_ragged_with_empty_requests_on_device_plan():
    say("device plan: ragged qo (incl. 0), kv 0, max_qo 17")
    qo = np.array([5, 0, 1, 17, 5, 2, 0, 5])
    ctx = np.array([100, 50, 0, 900, 3, 0, 10, 2000])
    b = make_verify_batch(8, 0, 0, 0, 32, 8, 128, 16, dtype=torch.bfloat16, seed=77, qo_lens=qo,
                          ctx=ctx).to(DEV)
    w = wrapper()
    device_plan(w, b, 17)
    out, lse = w.run(torch.cat([b.q, torch.zeros((8 * 17 - b.q.shape[0], 32, 128),
                                                 dtype=b.q.dtype, device=DEV)]), b.cache,
                     return_lse=True)
    compare_schedule(w, b, 17)
    n = b.q.shape[0]
    ref, ref_lse = oracle(b, "causal")
    check(out[:n], ref, lse[:n], ref_lse)


def test_tree_and_streaming_on_device_plan():
    say("device plan: 32-node trees, then a sink+window view")
    b = make_verify_batch(12, 100, 3000, 32, 32, 8, 128, 16, dtype=torch.bfloat16, seed=81,
                          tree_nodes=32).to(DEV)
    w = wrapper()
    words = torch.from_numpy(b.mask_words.view(np.int32)).to(DEV)
    device_plan(w, b, 32, causal=False, tree_mask_words=words)
    out, lse = run_lse(w, b)
    compare_schedule(w, b, 32, mode=2)
    qo = np.diff(b.qo_indptr.cpu().numpy())
    flat = []
    for r, L in enumerate(b.kv_lens):
        wd = b.mask_words[b.qo_indptr[r].item(): b.qo_indptr[r + 1].item()]
        blk = ((wd[:, None].astype(np.uint64) >> np.arange(qo[r], dtype=np.uint64)) & 1).astype(bool)
        flat.append(np.concatenate([np.ones((qo[r], L - qo[r]), bool), blk], 1).ravel())
    ref, ref_lse = oracle(b, "custom", custom_mask=np.concatenate(flat))
    check(out, ref, lse, ref_lse)

    s = make_verify_batch(6, 2000, 9000, 1, 32, 8, 128, 16, dtype=torch.bfloat16, seed=82).to(DEV)
    w2 = wrapper()
    device_plan(w2, s, 1, sink_tokens=64, window_tokens=512)
    out, lse = run_lse(w2, s)
    compare_schedule(w2, s, 1, mode=3, sink=64, window=512)
    ref, ref_lse = oracle(s, "streaming", sink=64, window=512)
    check(out, ref, lse, ref_lse)


def test_graph_replays_follow_the_page_table():
    """plan(on_device) + run captured once; three page-table states written into the
    captured input buffers in place; every replay equals an eager run of the same
    state bit for bit and the oracle within tolerance."""
    say("graph capture of plan(on_device=True) + run, three page-table states")
    B, qo, H, Hkv, D, ps = 16, 5, 32, 8, 128, 16
    states = [make_verify_batch(B, 30, 2500, qo, H, Hkv, D, ps, dtype=torch.bfloat16, scale=0.5,
                                seed=900 + i) for i in range(3)]
    max_pages = max(int(s.kv_indptr[-1]) for s in states)
    # one cache holding every state's pages (each state's pages rebased past the others)
    caches, base = [], 0
    for s in states:
        s.kv_indices = s.kv_indices + base
        base += s.cache.shape[0]
        caches.append(s.cache)
    cache = torch.cat(caches).to(DEV)
    qo_buf = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    kvp_buf = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    last_buf = torch.zeros(B, dtype=torch.int32, device=DEV)
    idx_buf = torch.zeros(max_pages, dtype=torch.int32, device=DEV)
    q_buf = torch.zeros((B * qo, H, D), dtype=torch.bfloat16, device=DEV)
    out_buf = torch.zeros_like(q_buf)

    def load(s):
        qo_buf.copy_(s.qo_indptr)
        kvp_buf.copy_(s.kv_indptr)
        last_buf.copy_(s.kv_last_page_len)
        idx_buf[: s.kv_indices.numel()].copy_(s.kv_indices)
        q_buf.copy_(s.q)

    w = wrapper(use_cuda_graph=True, paged_kv_indices_buf=idx_buf)
    load(states[0])
    step = lambda: (w.plan(qo_buf, kvp_buf, idx_buf, last_buf, H, Hkv, D, ps, causal=True,
                           q_data_type=torch.bfloat16, on_device=True, max_qo_len=qo),
                    w.run(q_buf, cache, out=out_buf))
    s_side = torch.cuda.Stream()
    s_side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_side):
        step()  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s_side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for rep in range(2):
        for i, s in enumerate(states):
            load(s)
            g.replay()
            torch.cuda.synchronize()
            got = out_buf.clone()
            eager = wrapper()
            sd = s.to(DEV)
            sd.cache = cache
            device_plan(eager, sd, qo)
            ref = eager.run(sd.q, cache)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"replay {rep} state {i} differs from the eager run"
            if rep == 0:
                s_cpu = s
                s_cpu.cache = cache.cpu()
                check(got, oracle(s_cpu, "causal")[0])


def test_malformed_table_reports_and_writes_nothing():
    say("device plan with a request above max_qo_len: error code, empty schedule")
    b = make_verify_batch(4, 10, 200, 6, 32, 8, 128, 16, dtype=torch.bfloat16, seed=5).to(DEV)
    w = wrapper()
    device_plan(w, b, 5)  # 6 tokens per request > 5
    sentinel = torch.full((4 * 5, 32, 128), 7.0, dtype=torch.bfloat16, device=DEV)
    w.run(b.q[:20].contiguous(), b.cache, out=sentinel)
    torch.cuda.synchronize()
    assert w.device_plan_error() == OS.ERR_UNSUPPORTED
    assert (sentinel == 7.0).all()
    got = blob_of(w)
    assert len(got["segments"]) == 0 and (got["seg_indptr"] == 0).all() and got["dyn"][0] == 0
