"""GPU parity of verify attention (through the C ABI) against the fp32 oracle.

Tolerance (bf16/fp16 inputs; the oracle sees the same rounded inputs in fp32):
|gpu - oracle| <= 2e-2 + 2e-2 * |oracle|  — the bound BASELINE.json's north star sets —
and, so that small outputs are checked too, max |gpu - oracle| <= 2e-2 * max |oracle| and
relative L2 error <= 1e-2; lse within 5e-3 where compared.  The benchmark shapes run with
planted keys and guards that show the check rejects a missing mask, a dropped tile and
zeros on the same inputs (tests/attn_parity.py).
"""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import masks as M
from batchspec_amd.workloads import config2, config3, config4, make_verify_batch
from oracle import attention as OA
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
ATOL = RTOL = 2e-2
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def oracle_out(b, mode, **kw):
    return OA.verify_attention(b.q.float().cpu().numpy(), b.cache.float().cpu().numpy(),
                               b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                               b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(),
                               b.page_size, mode=mode, **kw)


def run_gpu(b, causal=True, workspace_mb=256, **plan_kw):
    ws = torch.empty(workspace_mb << 20, dtype=torch.uint8, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
           b.num_kv_heads, b.head_dim, b.page_size, causal=causal, q_data_type=b.q.dtype, **plan_kw)
    out = w.run(b.q, b.cache)
    torch.cuda.synchronize()
    return out, w


def check(got, ref):
    """The north-star bound plus the normalised ones (tests/attn_parity.py)."""
    AP.check(got, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,Hq,Hkv", [(64, 8, 2), (128, 32, 8), (128, 8, 8), (64, 16, 2)])
def test_causal_small(dtype, D, Hq, Hkv):
    say(f"causal small dtype={dtype} D={D} H={Hq}/{Hkv}")
    b = make_verify_batch(4, 64, 256, 5, Hq, Hkv, D, 16, dtype=dtype, seed=1001).to(DEV)
    out, _ = run_gpu(b)
    check(out, oracle_out(b, "causal"))


def test_config1_shape_fp32_inputs_cast():
    say("config1 inputs cast to bf16")
    b = make_verify_batch(4, 64, 256, 5, 8, 2, 64, 16, dtype=torch.float32, seed=1001)
    b.q, b.cache = b.q.to(torch.bfloat16), b.cache.to(torch.bfloat16)
    b = b.to(DEV)
    out, _ = run_gpu(b)
    check(out, oracle_out(b, "causal"))


@pytest.mark.parametrize("ps", [1, 8, 16, 32, 64])
def test_page_sizes(ps):
    say(f"page size {ps}")
    b = make_verify_batch(5, 30, 300, 5, 32, 8, 128, ps, dtype=torch.bfloat16, seed=ps,
                          extra_pages=7).to(DEV)
    out, _ = run_gpu(b)
    check(out, oracle_out(b, "causal"))


@pytest.mark.parametrize("qo", [1, 3, 8, 16, 40])
def test_query_lengths(qo):
    say(f"qo={qo}")
    b = make_verify_batch(6, 50, 900, qo, 32, 8, 128, 16, dtype=torch.bfloat16, seed=100 + qo).to(DEV)
    out, _ = run_gpu(b)
    check(out, oracle_out(b, "causal"))


# Shapes with several waves per kv head (query rows > 32), which share each K/V tile
# through LDS: (D, Hq, Hkv, qo, page size, dtype, ctx range, causal, waves per head).
SHARED_CASES = [
    (64, 32, 4, 12, 32, torch.float16, (100, 2000), True, 4),
    (64, 16, 2, 40, 16, torch.bfloat16, (50, 1500), True, 8),   # two query groups
    (128, 32, 8, 24, 64, torch.float16, (8000, 20000), True, 4),  # split + merge
    (128, 32, 8, 33, 16, torch.bfloat16, (40, 3000), False, 8),
    (128, 32, 8, 16, 16, torch.bfloat16, (1, 700), True, 2),
]


@pytest.mark.parametrize("case", range(len(SHARED_CASES)))
def test_shared_kv_tiles(case):
    D, Hq, Hkv, qo, ps, dtype, (lo, hi), causal, qb = SHARED_CASES[case]
    say(f"shared kv tiles D={D} H={Hq}/{Hkv} qo={qo} ps={ps} {dtype} ctx=[{lo},{hi}] causal={causal}")
    b = make_verify_batch(5, lo, hi, qo, Hq, Hkv, D, ps, dtype=dtype, scale=0.5,
                          seed=300 + case).to(DEV)
    out, w = run_gpu(b, causal=causal)
    assert w.plan_info.shared_kv_tiles == 1 and w.plan_info.qblocks_per_cta == qb
    check(out, oracle_out(b, "causal" if causal else "none"))


def test_ragged_mixed_batch_with_empty_requests():
    say("ragged qo/ctx incl. qo=0 and kv=0")
    qo = np.array([5, 0, 1, 17, 5, 2, 0, 5])
    ctx = np.array([100, 40, 0, 700, 3000, 0, 5, 31])
    b = make_verify_batch(8, 0, 0, 0, 32, 8, 128, 16, dtype=torch.bfloat16, seed=7, qo_lens=qo,
                          ctx=ctx).to(DEV)
    out, _ = run_gpu(b)
    check(out, oracle_out(b, "causal"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_continuous_batching_mix(dtype):
    """The continuous-batching scheduler's mix (batchspec/backends/continuous/scheduler.py:
    189-204): prefill chunks up to 128 tokens, verify rows of k+1, decode rows and dummy
    1-token slots in one plan; 128 tokens x GQA 4 = 512 query rows per kv head."""
    say(f"continuous-batching mix: prefill chunks 128/64, verify 5, decode 1, {dtype}")
    qo = np.array([128, 5, 5, 1, 1, 64, 5, 1])
    ctx = np.array([0, 900, 2500, 4000, 0, 300, 17, 1])
    b = make_verify_batch(8, 0, 0, 0, 32, 8, 128, 16, dtype=dtype, scale=0.5, seed=19,
                          qo_lens=qo, ctx=ctx).to(DEV)
    out, w = run_gpu(b)
    assert w.plan_info.shared_kv_tiles == 1 and w.plan_info.num_qgroups == 2
    check(out, oracle_out(b, "causal"))


@pytest.mark.parametrize("ps", [1, 8])
def test_many_query_rows_on_small_pages(ps):
    """Pages under 16 tokens keep the per-wave kernel even with several query blocks per kv
    head: 32-node trees (128 rows per kv head) and 16-token causal drafts (64 rows)."""
    say(f"page size {ps}: 32-node trees, then 16-token causal drafts")
    b = make_verify_batch(5, 40, 1500, 32, 32, 8, 128, ps, dtype=torch.bfloat16, scale=0.5,
                          seed=40 + ps, tree_nodes=32).to(DEV)
    out, w = run_gpu(b, causal=False, tree_mask_words=b.mask_words)
    assert w.plan_info.shared_kv_tiles == 0 and w.plan_info.qrow_blocks == 4
    qo = np.diff(b.qo_indptr.cpu().numpy())
    flat = []
    for r, L in enumerate(b.kv_lens):
        wd = b.mask_words[b.qo_indptr[r].item(): b.qo_indptr[r + 1].item()]
        blk = ((wd[:, None].astype(np.uint64) >> np.arange(qo[r], dtype=np.uint64)) & 1).astype(bool)
        flat.append(np.concatenate([np.ones((qo[r], L - qo[r]), bool), blk], 1).ravel())
    check(out, oracle_out(b, "custom", custom_mask=np.concatenate(flat)))
    c = make_verify_batch(6, 10, 900, 16, 32, 8, 128, ps, dtype=torch.float16, scale=0.5,
                          seed=50 + ps).to(DEV)
    out, w = run_gpu(c)
    assert w.plan_info.shared_kv_tiles == 0
    check(out, oracle_out(c, "causal"))


def test_non_causal():
    say("non-causal")
    b = make_verify_batch(5, 10, 500, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=3).to(DEV)
    out, _ = run_gpu(b, causal=False)
    check(out, oracle_out(b, "none"))


def test_long_context_split_and_merge():
    say("long context split/merge, planted keys at segment boundaries")
    b = make_verify_batch(3, 20000, 40000, 5, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=11).to(DEV)
    out, w = run_gpu(b)
    assert w.plan_info.num_split_requests == 3
    check(out, oracle_out(b, "causal"))
    AP.plant_keys(b, "causal", plan_blob=w.plan_blob, plan=w.plan_info, seed=11)
    out, lse = w.run(b.q, b.cache, return_lse=True)
    ref = AP.oracle_per_request(b, "causal")[None]
    AP.check(out, ref[0], lse, ref[1])


def test_repeated_runs_reuse_the_plan():
    """One plan serves any number of runs; the split-and-merge path is deterministic, so
    back-to-back runs give identical results."""
    say("repeated runs of one plan (split requests)")
    b = make_verify_batch(6, 3000, 9000, 5, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=12).to(DEV)
    out, w = run_gpu(b)
    assert w.plan_info.num_split_requests == 6
    check(out, oracle_out(b, "causal"))
    for i in range(5):
        again = w.run(b.q, b.cache)
        torch.cuda.synchronize()
        assert torch.equal(again, out), f"run {i}"


def test_lse_output():
    say("lse")
    b = make_verify_batch(4, 100, 3000, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=5).to(DEV)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws)
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, 32, 8, 128, 16,
           causal=True, q_data_type=torch.bfloat16)
    out, lse = w.run(b.q, b.cache, return_lse=True)
    ref, ref_lse = OA.verify_attention(b.q.float().cpu().numpy(), b.cache.float().cpu().numpy(),
                                       b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                                       b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(),
                                       16, mode="causal", return_lse=True)
    check(out, ref)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=2e-2, rtol=1e-3)


def test_tree_mask_words():
    say("tree mask, 32 nodes")
    b = make_verify_batch(6, 100, 2000, 32, 32, 8, 128, 16, dtype=torch.bfloat16, seed=21,
                          tree_nodes=32).to(DEV)
    out, _ = run_gpu(b, causal=False, tree_mask_words=b.mask_words)
    # dense mask per request: all prefix columns + the ancestor block
    flat = []
    qo = np.diff(b.qo_indptr.cpu().numpy())
    for r, L in enumerate(b.kv_lens):
        w = b.mask_words[b.qo_indptr[r].item(): b.qo_indptr[r + 1].item()]
        blk = ((w[:, None].astype(np.uint64) >> np.arange(qo[r], dtype=np.uint64)) & 1).astype(bool)
        flat.append(np.concatenate([np.ones((qo[r], L - qo[r]), bool), blk], 1).ravel())
    check(out, oracle_out(b, "custom", custom_mask=np.concatenate(flat)))


def test_mtp_custom_mask_via_plan():
    say("MTP (k+1)^2 custom mask through plan(custom_mask=...)")
    k = 4
    S = (k + 1) ** 2
    b = make_verify_batch(4, 20, 400, S, 32, 8, 128, 16, dtype=torch.bfloat16, seed=31).to(DEV)
    flat = M.mtp_verify_custom_mask(b.ctx.tolist(), k, device=DEV)
    out, _ = run_gpu(b, causal=False, custom_mask=flat)
    check(out, oracle_out(b, "custom", custom_mask=flat.cpu().numpy()))


def test_streaming_sink_window_view():
    say("sink+window view")
    b = make_verify_batch(4, 3000, 9000, 1, 32, 8, 128, 16, dtype=torch.bfloat16, seed=41).to(DEV)
    out, _ = run_gpu(b, causal=True, sink_tokens=64, window_tokens=512)
    check(out, oracle_out(b, "streaming", sink=64, window=512))


def test_page_permutation_invariance_bitwise():
    say("page permutation invariance")
    b = make_verify_batch(6, 500, 3000, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=51,
                          extra_pages=11).to(DEV)
    out1, _ = run_gpu(b)
    P = b.cache.shape[0]
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(1)).to(DEV)
    cache2 = torch.empty_like(b.cache)
    cache2[perm] = b.cache
    b.cache, b.kv_indices = cache2, perm[b.kv_indices.long()].to(torch.int32)
    out2, _ = run_gpu(b)
    assert torch.equal(out1, out2)


def test_tuple_cache_layout_matches_combined():
    say("tuple (k, v) cache")
    b = make_verify_batch(4, 100, 900, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=61).to(DEV)
    out1, w = run_gpu(b)
    k, v = b.cache[:, 0].contiguous(), b.cache[:, 1].contiguous()
    out2 = w.run(b.q, (k, v))
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_graph_capture_replays():
    say("hip graph capture of run()")
    b = make_verify_batch(8, 200, 3000, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=71).to(DEV)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    idx_buf = torch.empty(b.kv_indices.numel() + 64, dtype=torch.int32, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD", use_cuda_graph=True,
                                                paged_kv_indices_buf=idx_buf)
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, 32, 8, 128, 16,
           causal=True, q_data_type=torch.bfloat16)
    out = torch.empty_like(b.q)
    eager = w.run(b.q, b.cache).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w.run(b.q, b.cache, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w.run(b.q, b.cache, out=out)
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


# ---- the benchmark shapes, with checks that can fail (tests/attn_parity.py) -----------

def _host_plan_run(b, causal=True, lse=True, **plan_kw):
    ws = torch.empty(512 << 20, dtype=torch.uint8, device=DEV)
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
           b.num_kv_heads, b.head_dim, b.page_size, causal=causal, q_data_type=b.q.dtype, **plan_kw)
    return w


def _run(w, b):
    out, lse = w.run(b.q, b.cache, return_lse=True)
    torch.cuda.synchronize()
    return out, lse


def test_config2_full_size():
    """Config 2 (B=64, ctx 1k-4k, 5 causal queries, 32/8 heads, D=128) on the plan the
    bench times: plain inputs, then planted keys at the draft block, hidden next draft
    tokens, segment and tile boundaries; guards show the check rejects a missing mask,
    a dropped last tile and zeros on these very inputs."""
    say("config 2 full size: plain inputs")
    b = config2(device=DEV)
    w = _host_plan_run(b)
    out, lse = _run(w, b)
    ref = AP.oracle_per_request(b, "causal")[None]
    e, m = AP.check(out, ref[0], lse, ref[1])
    say(f"  plain: max err {e:.3g} (max|ref| {m:.3g}), split requests {w.plan_info.num_split_requests}")
    say("config 2 full size: planted keys")
    AP.plant_keys(b, "causal", plan_blob=w.plan_blob, plan=w.plan_info, seed=2)
    out, lse = _run(w, b)
    res = AP.oracle_per_request(b, "causal", mutations=("nomask", "droplast"))
    e, m = AP.check(out, res[None][0], lse, res[None][1])
    say(f"  planted: max err {e:.3g} (max|ref| {m:.3g})")
    AP.assert_discriminates(res[None], [("no mask", *res["nomask"]),
                                        ("last tile dropped", *res["droplast"]),
                                        ("zeros", np.zeros_like(res[None][0]), None)])


def test_config4_tree_full_size():
    """Config 4 (B=32 trees of 32 nodes, ctx 2k-8k) on the shared-tile kernel the bench
    times, plain and with planted keys (ancestor and non-ancestor nodes, segment and
    tile boundaries); guards: no tree mask, dropped last tile."""
    say("config 4 full size: plain inputs")
    b = config4(device=DEV)
    w = _host_plan_run(b, causal=False, tree_mask_words=b.mask_words)
    assert w.plan_info.shared_kv_tiles == 1
    out, lse = _run(w, b)
    ref = AP.oracle_per_request(b, "tree")[None]
    e, m = AP.check(out, ref[0], lse, ref[1])
    say(f"  plain: max err {e:.3g} (max|ref| {m:.3g})")
    say("config 4 full size: planted keys")
    AP.plant_keys(b, "tree", plan_blob=w.plan_blob, plan=w.plan_info, seed=4)
    out, lse = _run(w, b)
    res = AP.oracle_per_request(b, "tree", mutations=("nomask", "droplast"))
    e, m = AP.check(out, res[None][0], lse, res[None][1])
    say(f"  planted: max err {e:.3g} (max|ref| {m:.3g})")
    AP.assert_discriminates(res[None], [("no tree mask", *res["nomask"]),
                                        ("last tile dropped", *res["droplast"])])


def test_config3b_full_size_split_and_merge():
    """Config 3b in full (B=32, ctx 32k-64k, 5 causal queries; every request split over
    several workgroups and merged), with planted keys at segment boundaries; the oracle
    gathers each request's pages on the device.  Guards: zeros, no mask, dropped tile."""
    say("config 3b full size (B=32, 32k-64k): planted keys")
    b = config3(device=DEV)
    w = _host_plan_run(b)
    assert w.plan_info.num_split_requests == 32
    AP.plant_keys(b, "causal", plan_blob=w.plan_blob, plan=w.plan_info, seed=3)
    out, lse = _run(w, b)
    res = AP.oracle_per_request(b, "causal", mutations=("nomask", "droplast"), progress=8)
    e, m = AP.check(out, res[None][0], lse, res[None][1])
    say(f"  planted: max err {e:.3g} (max|ref| {m:.3g}), segments {w.plan_info.num_segments}")
    AP.assert_discriminates(res[None], [("zeros", np.zeros_like(res[None][0]), None),
                                        ("no mask", *res["nomask"]),
                                        ("last tile dropped", *res["droplast"])])


def test_config3b_plain_inputs_normalised():
    """Config 3b's plain inputs (|O| ~ 0.01): the normalised bound (max err <= 2e-2
    max|ref|, relative L2 <= 1e-2) and the lse carry the check; 8 requests."""
    say("config 3b plain inputs, 8 requests")
    b = config3(device=DEV, batch=8)
    w = _host_plan_run(b)
    out, lse = _run(w, b)
    ref = AP.oracle_per_request(b, "causal")[None]
    e, m = AP.check(out, ref[0], lse, ref[1])
    say(f"  plain: max err {e:.3g} (max|ref| {m:.3g}, ratio {e / m:.3g})")
    AP.assert_discriminates(ref, [("zeros", np.zeros_like(ref[0]), None)])


def test_split_partials_against_an_unsplit_run():
    """What storing split-KV partials in the input dtype costs: config 3b's plain inputs
    (4 requests of 32k-64k tokens) on the default plan, every request split and merged,
    against a one-workgroup plan that splits nothing; both against the oracle."""
    say("config 3b plain inputs, 4 requests: split plan vs unsplit plan")
    b = config3(device=DEV, batch=4)
    w = _host_plan_run(b)
    assert w.plan_info.num_split_requests == 4
    split, _ = _run(w, b)
    w1 = bsx.BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8,
                                                             device=DEV), "NHD")
    w1._num_cus = 1  # a persistent grid of one workgroup: no request is split
    w1.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
            b.num_kv_heads, b.head_dim, b.page_size, causal=True, q_data_type=b.q.dtype)
    assert w1.plan_info.num_ctas == 1 and w1.plan_info.num_split_requests == 0
    whole, _ = _run(w1, b)
    ref = AP.oracle_per_request(b, "causal")[None]
    m = float(np.abs(ref[0]).max())
    d = (split.float() - whole.float()).abs().max().item()
    e_split = float(np.abs(split.float().cpu().numpy() - ref[0]).max())
    e_whole = float(np.abs(whole.float().cpu().numpy() - ref[0]).max())
    say(f"  max|ref| {m:.3g}; max|split - unsplit| {d:.3g} ({d / m:.3%}); vs oracle: "
        f"split {e_split / m:.3%}, unsplit {e_whole / m:.3%}; "
        f"{w.plan_info.num_segments} segments")
    AP.check(split, ref[0])
    AP.check(whole, ref[0])
    assert d <= 1e-2 * m


def test_config3a_sink_window_full_size():
    """Config 3a (B=32, one query over a 64-sink + 512-window view of 32k-64k tokens)
    with planted keys at the view's edges; guards: sink or window off by one/32."""
    say("config 3a full size: sink+window view, planted edges")
    d = make_verify_batch(32, 32768, 65536, 1, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=1003, device=DEV)
    w = _host_plan_run(d, causal=True, sink_tokens=64, window_tokens=512)
    AP.plant_keys(d, "streaming", seed=5, sink=64, window=512)
    out, lse = _run(w, d)
    ref = AP.oracle_per_request(d, "streaming", sink=64, window=512)[None]
    e, m = AP.check(out, ref[0], lse, ref[1])
    say(f"  planted: max err {e:.3g} (max|ref| {m:.3g})")
    bad = [(f"sink {s} window {wn}", *AP.oracle_per_request(d, "streaming", sink=s, window=wn)[None])
           for s, wn in ((63, 512), (64, 480))]
    AP.assert_discriminates(ref, bad)
