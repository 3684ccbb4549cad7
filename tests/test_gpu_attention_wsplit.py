"""The wave-split attention kernel (one workgroup per request and kv head, whose eight
waves split the request's visible tiles and merge in LDS), planned for at most 16 query
rows per kv head over views of at most 32 tiles when the (request, kv head) pairs number
between half the compute units and all of them and the planner's time model favours it:
config 3a's sink + window view, short views, short drafts.  Parity
against the fp32 oracle with the tolerance of tests/test_gpu_attention.py (and lse within
2e-2), planted keys at the waves' run boundaries with guards, and the fused KV append
equal to append + run bit for bit."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd.workloads import make_verify_batch
from oracle import attention as OA
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
WAVE_SPLIT = 2  # bsx_attn_plan_t.shared_kv_tiles of the wave-split kernel
WAVES = 8


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _plan(b, **kw):
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(
        torch.empty(256 << 20, dtype=torch.uint8, device=DEV), "NHD")
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
           b.num_kv_heads, b.head_dim, b.page_size, q_data_type=b.q.dtype, **kw)
    return w


def _oracle(b, mode, **kw):
    return OA.verify_attention(b.q.float().cpu().numpy(), b.cache.float().cpu().numpy(),
                               b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                               b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(),
                               b.page_size, mode=mode, return_lse=True, **kw)


def _check(b, w, mode, **kw):
    out, lse = w.run(b.q, b.cache, return_lse=True)
    torch.cuda.synchronize()
    ref, ref_lse = _oracle(b, mode, **kw)
    AP.check(out, ref)
    rows = np.asarray(ref_lse)
    np.testing.assert_allclose(lse.cpu().numpy(), rows, atol=2e-2, rtol=1e-3)
    return out


def _assert_wave_split(w):
    p = w.plan_info
    assert p.shared_kv_tiles == WAVE_SPLIT, "expected the wave-split plan"
    assert p.num_split_requests == 0 and p.num_partials == 0 and p.float_ws_bytes == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,Hq,Hkv,B", [(128, 32, 8, 32), (64, 16, 4, 64), (128, 8, 8, 24)])
def test_single_token_decode(dtype, D, Hq, Hkv, B):
    """Views of 1..10 tiles (under the wave count for most requests)."""
    say(f"wave split: one query token, {dtype} D={D} H={Hq}/{Hkv} B={B}")
    b = make_verify_batch(B, 1, 300, 1, Hq, Hkv, D, 16, dtype=dtype, seed=D + B).to(DEV)
    w = _plan(b, causal=True)
    _assert_wave_split(w)
    _check(b, w, "causal")


@pytest.mark.parametrize("qo", [2, 4])
def test_short_drafts_causal_and_non_causal(qo):
    """qo_len * group = 8 / 16 query rows per kv head: the causal limit inside the rows."""
    say(f"wave split: {qo} draft tokens, causal and non-causal")
    b = make_verify_batch(32, 30, 1000, qo, 32, 8, 128, 16, dtype=torch.bfloat16, seed=qo).to(DEV)
    w = _plan(b, causal=True)
    _assert_wave_split(w)
    _check(b, w, "causal")
    w2 = _plan(b, causal=False)
    _assert_wave_split(w2)
    _check(b, w2, "none")


def test_ragged_with_empty_requests_and_pages():
    """Requests with no query, no kv, fewer tiles than waves, and page sizes 16 / 32 / 64."""
    say("wave split: ragged lengths, empty requests, page sizes")
    rng = np.random.default_rng(3)
    qo = rng.integers(1, 5, 32)
    qo[[0, 3, 17, 30]] = 4
    qo[[4, 18, 31]] = 0
    ctx = rng.integers(0, 1000, 32)
    ctx[[5, 9]] = 0
    ctx[[11, 12]] = [1, 31]
    for ps in (16, 32, 64):
        b = make_verify_batch(32, 0, 0, 0, 32, 8, 128, ps, dtype=torch.bfloat16, seed=ps,
                              qo_lens=qo, ctx=ctx, extra_pages=5).to(DEV)
        w = _plan(b, causal=True)
        _assert_wave_split(w)
        _check(b, w, "causal")


@pytest.mark.parametrize("ctx", [(300, 600), (600, 1200), (3000, 9000)])
def test_sink_window_views(ctx):
    """Views without a gap (kv <= sink + window), with a gap, and long contexts."""
    say(f"wave split: 64-sink + 512-window views, ctx {ctx}")
    b = make_verify_batch(32, ctx[0], ctx[1], 1, 32, 8, 128, 16, dtype=torch.bfloat16,
                          seed=ctx[0]).to(DEV)
    w = _plan(b, causal=True, sink_tokens=64, window_tokens=512)
    _assert_wave_split(w)
    _check(b, w, "streaming", sink=64, window=512)


def test_not_planned_when_it_does_not_fit():
    """Fewer pairs than half the compute units, more pairs than units (short views, 36%
    slower on the wave split at 2048 pairs), ragged single-token views of up to 32 tiles
    that the time model gives to the split, more than 16 query rows per kv head, a view of
    more than 32 tiles, small pages: the split-KV schedule instead."""
    say("wave split: shapes that keep the split-KV schedule")
    cases = [
        make_verify_batch(8, 10, 300, 1, 32, 8, 128, 16, dtype=torch.bfloat16, seed=1),
        make_verify_batch(64, 50, 300, 1, 32, 8, 128, 16, dtype=torch.bfloat16, seed=5),
        make_verify_batch(16, 500, 1000, 1, 32, 8, 128, 16, dtype=torch.bfloat16, seed=6),
        make_verify_batch(64, 10, 900, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=2),
        make_verify_batch(64, 1100, 3000, 1, 32, 8, 128, 16, dtype=torch.bfloat16, seed=3),
        make_verify_batch(64, 10, 900, 1, 32, 8, 128, 8, dtype=torch.bfloat16, seed=4),
    ]
    for b in cases:
        b = b.to(DEV)
        w = _plan(b, causal=True)
        assert w.plan_info.shared_kv_tiles != WAVE_SPLIT
        _check(b, w, "causal")


def _wave_runs(b):
    """The waves' runs of tiles as segments (request, first tile, end tile, slot) of a
    causal view: wave w takes tiles [T w / 8, T (w + 1) / 8) of a request's T tiles."""
    segs = []
    for r, L in enumerate(b.kv_lens):
        T = -(-int(L) // 32)
        for w in range(WAVES):
            t0, t1 = T * w // WAVES, T * (w + 1) // WAVES
            if t1 > t0:
                segs.append((r, t0, t1, -1))
    return np.array(segs, dtype=np.int64)


def test_planted_keys_at_wave_boundaries():
    """Keys planted where the waves' runs meet and at the draft tokens (4 per request, so
    the causal mask hides the later ones); guards show the check rejects a missing mask, a
    dropped last tile and zeros on these inputs."""
    say("wave split: planted keys at the waves' run boundaries")
    b = make_verify_batch(32, 200, 1000, 4, 32, 8, 128, 16, dtype=torch.bfloat16, scale=0.5,
                          seed=77, device=DEV)
    w = _plan(b, causal=True)
    _assert_wave_split(w)
    AP.plant_keys(b, "causal", seed=9, segments=_wave_runs(b))
    out, lse = w.run(b.q, b.cache, return_lse=True)
    torch.cuda.synchronize()
    res = AP.oracle_per_request(b, "causal", mutations=("nomask", "droplast"))
    e, m = AP.check(out, res[None][0], lse, res[None][1])
    say(f"  planted: max err {e:.3g} (max|ref| {m:.3g})")
    AP.assert_discriminates(res[None], [("no mask", *res["nomask"]),
                                        ("dropped last tile", *res["droplast"]),
                                        ("zeros", np.zeros_like(res[None][0]), None)])


def test_fused_append_equals_append_then_run():
    say("wave split: fused KV append equals append + run")
    for kw, s in ((dict(causal=True), make_verify_batch(32, 10, 900, 4, 32, 8, 128, 16,
                                                       dtype=torch.bfloat16, seed=21)),
                  (dict(causal=True, sink_tokens=64, window_tokens=512),
                   make_verify_batch(32, 2000, 9000, 1, 32, 8, 128, 16, dtype=torch.bfloat16,
                                     seed=22))):
        s = s.to(DEV)
        w = _plan(s, **kw)
        _assert_wave_split(w)
        c_two = s.cache.clone()
        bsx.append_kv(s.k_new, s.v_new, s.qo_indptr, c_two, s.kv_indptr, s.kv_indices,
                      s.kv_last_page_len)
        o2, l2 = w.run(s.q, c_two, return_lse=True)
        c_one = s.cache.clone()
        o1, l1 = w.run(s.q, c_one, return_lse=True, append_key=s.k_new, append_value=s.v_new)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(l1, l2) and torch.equal(c_one, c_two)


@pytest.mark.parametrize("dtype,D,Hq,Hkv", [(torch.float16, 128, 32, 8), (torch.bfloat16, 64, 16, 8),
                                            (torch.float16, 64, 32, 8)])
def test_sink_window_dtypes_and_head_dims(dtype, D, Hq, Hkv):
    say(f"wave split: sink + window view, {dtype} D={D} H={Hq}/{Hkv}")
    b = make_verify_batch(32, 2000, 6000, 1, Hq, Hkv, D, 16, dtype=dtype, seed=D + Hq).to(DEV)
    w = _plan(b, causal=True, sink_tokens=64, window_tokens=512)
    _assert_wave_split(w)
    _check(b, w, "streaming", sink=64, window=512)


def test_captured_run_replays():
    """run() on a wave-split plan captured in a CUDA graph: each replay, with new q and
    cache contents written between replays, equals the eager run on the same inputs."""
    say("wave split: captured run() replays")
    b = make_verify_batch(32, 100, 1000, 2, 32, 8, 128, 16, dtype=torch.bfloat16, seed=5).to(DEV)
    w = _plan(b, causal=True)
    _assert_wave_split(w)
    q = b.q.clone()
    cache = b.cache.clone()
    out = torch.empty_like(q)
    w.run(q, cache, out=out)  # warm up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w.run(q, cache, out=out)
    gen = torch.Generator(device="cpu").manual_seed(11)
    for rep in range(4):
        q.copy_((torch.randn(q.shape, generator=gen) * 0.5).to(q.dtype))
        cache.copy_((torch.randn(cache.shape, generator=gen) * 0.5).to(cache.dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = w.run(q, cache)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep} differs from the eager run"


@pytest.mark.parametrize("qo", [1, 4])
def test_head_dim_64_long_views(qo):
    """Head dim 64 over views of up to 32 tiles (four per wave): the planner gives them to
    the wave split at 128..256 pairs, single tokens and 4-token drafts alike."""
    say(f"wave split: head dim 64, views of up to 32 tiles, {qo} query tokens")
    for B, seed in ((16, 60 + qo), (32, 70 + qo)):
        b = make_verify_batch(B, 30, 1000, qo, 32, 8, 64, 16, dtype=torch.bfloat16,
                              seed=seed).to(DEV)
        w = _plan(b, causal=True)
        _assert_wave_split(w)
        _check(b, w, "causal")
