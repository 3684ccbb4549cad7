"""The layer's KV update fused with its attention (run(..., append_key=, append_value=),
bsx_attn_run_append) against the two calls it replaces: StandardKVCache.update with
kv_append_indptr = qo_indptr (batchspec/models/modules/kv_cache.py:47-84, called at
batchspec/models/modules/attention/standard.py:63-66) and then run() (standard.py:69).
Outputs, lse and the whole cache must be equal bit for bit, over host and device plans,
the per-wave kernel with one and two row tiles, the shared-tile kernel, pages below 16
tokens, several query groups per kv head (workgroups writing the same rows), ragged
batches whose appended rows cross tile and page boundaries, split requests, causal / tree /
sink+window masks and both 16-bit types; and the eager result is checked against the fp32
oracle.  The starting cache holds random rows in the appended slots, so a read of a slot
before its write would show."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd.workloads import config2, make_verify_batch
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _wrapper(b, on_device=False, max_qo=None, **kw):
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(
        torch.empty(256 << 20, dtype=torch.uint8, device=DEV), "NHD")
    extra = dict(on_device=True, max_qo_len=max_qo) if on_device else {}
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
           b.num_kv_heads, b.head_dim, b.page_size, q_data_type=b.q.dtype, **extra, **kw)
    return w


def _both(b, w, q=None, k=None, v=None):
    """(out, lse, cache) of append-then-run and of the fused call, from the same cache."""
    q = b.q if q is None else q
    k = b.k_new if k is None else k
    v = b.v_new if v is None else v
    c_two = b.cache.clone()
    bsx.append_kv(k, v, b.qo_indptr, c_two, b.kv_indptr, b.kv_indices, b.kv_last_page_len)
    o2, l2 = w.run(q, c_two, return_lse=True)
    c_one = b.cache.clone()
    o1, l1 = w.run(q, c_one, return_lse=True, append_key=k, append_value=v)
    torch.cuda.synchronize()
    return (o1, l1, c_one), (o2, l2, c_two)


def _equal(got, want, what):
    for g, x, n in zip(got, want, ("out", "lse", "cache")):
        assert torch.equal(g, x), f"{what}: {n} differs from append + run"


def test_config2_fused_append_equals_append_then_run():
    say("fused append + attention, config 2 (host plan, then device plan)")
    b = config2(device=DEV)
    w = _wrapper(b, causal=True)
    got, want = _both(b, w)
    _equal(got, want, "config 2 host plan")
    ref = AP.oracle_per_request(_with_cache(b, want[2]), "causal")[None]
    e, m = AP.check(got[0], ref[0], got[1], ref[1])
    say(f"  vs oracle: max err {e:.3g} (max|ref| {m:.3g})")
    wd = _wrapper(b, causal=True, on_device=True, max_qo=5)
    got, want = _both(b, wd)
    _equal(got, want, "config 2 device plan")


def _with_cache(b, cache):
    c = b.to(DEV)
    c.cache = cache
    return c


@pytest.mark.parametrize("hq,hkv,dtype", [(32, 8, torch.bfloat16), (8, 8, torch.float16),
                                          (28, 4, torch.bfloat16)])
def test_ragged_appends_across_tiles_pages_and_splits(hq, hkv, dtype):
    """qo lengths up to 17 with contexts placing the appended rows across 32-token tile
    and 16-token page boundaries; long requests split over several workgroups."""
    say(f"fused append, ragged: H={hq}/{hkv} {dtype}")
    qo = np.array([5, 1, 17, 0, 3, 5, 9, 2])
    ctx = np.array([27, 60, 15, 40, 8000, 12000, 1, 31])
    b = make_verify_batch(8, 0, 0, 0, hq, hkv, 128, 16, dtype=dtype, scale=0.5, seed=hq + hkv,
                          qo_lens=qo, ctx=ctx, device=DEV)
    w = _wrapper(b, causal=True)
    assert w.plan_info.num_split_requests > 0
    got, want = _both(b, w)
    _equal(got, want, "ragged causal")
    ref = AP.oracle_per_request(_with_cache(b, want[2]), "causal")[None]
    AP.check(got[0], ref[0], got[1], ref[1])


def test_tree_small_pages_and_query_groups():
    say("fused append on the shared-tile kernel (trees), on 8-token pages, and with several "
        "query groups per kv head")
    t = make_verify_batch(6, 100, 3000, 32, 32, 8, 128, 16, dtype=torch.bfloat16, seed=8,
                          tree_nodes=32, device=DEV)
    wt = _wrapper(t, causal=False, tree_mask_words=t.mask_words)
    assert wt.plan_info.shared_kv_tiles == 1
    got, want = _both(t, wt)
    _equal(got, want, "tree")
    s = make_verify_batch(5, 20, 900, 5, 32, 8, 128, 8, dtype=torch.bfloat16, seed=9, device=DEV)
    ws = _wrapper(s, causal=True)
    got, want = _both(s, ws)
    _equal(got, want, "page size 8")
    for ps in (16, 8):  # 80 drafts x group 4 = 320 rows: two query groups per kv head
        d = make_verify_batch(4, 200, 3000, 80, 32, 8, 128, ps, dtype=torch.bfloat16,
                              seed=11 + ps, device=DEV)
        wd = _wrapper(d, causal=True)
        assert wd.plan_info.num_qgroups > 1
        got, want = _both(d, wd)
        _equal(got, want, f"two query groups, page size {ps}")
        ref = AP.oracle_per_request(_with_cache(d, want[2]), "causal")[None]
        AP.check(got[0], ref[0], got[1], ref[1])


def test_streaming_view_with_append():
    say("fused append with a sink + window view")
    s = make_verify_batch(6, 2000, 9000, 1, 32, 8, 128, 16, dtype=torch.bfloat16, seed=10,
                          device=DEV)
    w = _wrapper(s, causal=True, sink_tokens=64, window_tokens=512)
    got, want = _both(s, w)
    _equal(got, want, "sink + window")


def test_append_arguments_are_checked():
    b = make_verify_batch(2, 40, 60, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=3, device=DEV)
    w = _wrapper(b, causal=True)
    with pytest.raises(ValueError):
        w.run(b.q, b.cache, append_key=b.k_new)
    with pytest.raises(ValueError):
        w.run(b.q, b.cache, append_key=b.k_new[:3], append_value=b.v_new[:3])
    with pytest.raises(ValueError):
        w.run(b.q, b.cache, append_key=b.k_new.float(), append_value=b.v_new.float())
