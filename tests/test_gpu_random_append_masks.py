"""Randomized shapes for the fused KV update and the custom masks: batch sizes 1-12, query
lengths 0-40 (empty requests included), contexts 0-3000 (empty and sub-page ones
included), page sizes 1-64, GQA groups 1-7, head dims 64 and 128, both 16-bit types, and
the mask modes causal, none, a random general custom mask and a tree-form custom mask.

Every case checks the fused call (run(..., append_key=, append_value=)) against the append
followed by run() bit for bit (output, lse and the whole cache), and the result against
the fp32 oracle with the north-star bound plus the normalised bounds (tests/attn_parity.py)
on the appended cache.  The oracle applies each mask exactly as FlashInfer's plan() takes
it (the flattened boolean mask, request by request)."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import _lib
from batchspec_amd.workloads import make_verify_batch
from oracle import attention as OA
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
HEADS = [(32, 8), (8, 2), (16, 16), (28, 4)]
PAGES = [1, 4, 8, 16, 32, 64]
MODES = ["causal", "none", "general", "tree"]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 13))
    mode = MODES[seed % 4]
    qmax = 32 if mode == "tree" else 40
    qo = rng.integers(0, qmax + 1, size=B)
    qo[rng.random(B) < 0.15] = 0
    ctx = rng.integers(0, 3001, size=B)
    small = rng.random(B) < 0.3
    ctx[small] = rng.integers(0, 40, size=int(small.sum()))
    hq, hkv = HEADS[int(rng.integers(len(HEADS)))]
    D = 64 if rng.random() < 0.4 else 128
    ps = PAGES[int(rng.integers(len(PAGES)))]
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float16
    return rng, B, mode, qo, ctx, hq, hkv, D, ps, dtype


def _mask(rng, mode, qo, kv):
    parts = []
    for q, k in zip(qo, kv):
        if mode == "general":
            m = rng.random((q, k)) < 0.6
        else:  # tree form: the prefix visible, a random block over the last q columns
            m = np.ones((q, k), bool)
            if q:
                m[:, k - q:] = rng.random((q, q)) < 0.5
        parts.append(m.ravel())
    return np.concatenate(parts) if parts else np.zeros(0, bool)


@pytest.mark.parametrize("seed", range(24))
def test_random_fused_append_and_masks(seed):
    rng, B, mode, qo, ctx, hq, hkv, D, ps, dtype = _case(seed)
    say(f"case {seed}: B={B} mode={mode} qo={qo.tolist()} H={hq}/{hkv} D={D} page={ps} {dtype}")
    b = make_verify_batch(B, 0, 0, 0, hq, hkv, D, ps, dtype=dtype, scale=1.0, seed=seed,
                          qo_lens=qo, ctx=ctx, device=DEV)
    kv = b.kv_lens
    kw = {}
    omode, omask = mode, None
    if mode == "causal":
        kw["causal"] = True
    elif mode == "none":
        kw["causal"] = False
    else:
        omask = _mask(rng, mode, qo, kv)
        kw = dict(causal=False, custom_mask=torch.from_numpy(omask).to(DEV))
        omode = "custom"
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(
        torch.empty(64 << 20, dtype=torch.uint8, device=DEV), "NHD")
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, hq, hkv, D, ps,
           q_data_type=dtype, **kw)
    if mode == "tree":
        assert w.plan_info.mask_mode == _lib.MASK_TREE
    if mode == "general":
        off = np.concatenate([[0], np.cumsum(qo * kv)])
        tree_form = all(q <= 32 and np.all(omask[off[r]: off[r + 1]].reshape(q, k)[:, : k - q])
                        for r, (q, k) in enumerate(zip(qo, kv)))
        want = _lib.MASK_TREE if tree_form else _lib.MASK_CUSTOM
        assert w.plan_info.mask_mode == want
    c_two = b.cache.clone()
    bsx.append_kv(b.k_new, b.v_new, b.qo_indptr, c_two, b.kv_indptr, b.kv_indices,
                  b.kv_last_page_len)
    o2, l2 = w.run(b.q, c_two, return_lse=True)
    c_one = b.cache.clone()
    o1, l1 = w.run(b.q, c_one, return_lse=True, append_key=b.k_new, append_value=b.v_new)
    torch.cuda.synchronize()
    assert torch.equal(c_one, c_two), "cache differs from append + run"
    assert torch.equal(o1, o2), "output differs from append + run"
    assert torch.equal(l1, l2), "lse differs from append + run"
    if int(qo.sum()) == 0:
        return
    ref = OA.verify_attention(b.q.float().cpu().numpy(), c_two.float().cpu().numpy(),
                              b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                              b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(), ps,
                              mode=omode, custom_mask=omask, return_lse=True)
    AP.check(o1, ref[0], l1, ref[1])
