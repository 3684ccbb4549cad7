"""plan(custom_mask=...) with masks packed on the device (bsx_custom_mask_prepare) against
the fp32 oracle, which applies the flattened boolean mask exactly as FlashInfer's plan()
takes it (sum(qo_len * kv_len) entries, request by request; the MTP engine's call at
batchspec/backends/mtp_engine.py:399-432).

* The packed bits and tree words are compared with numpy's own packbits and a direct
  reading of the mask (bit-exact), for an unaligned mask and a malformed request.
* The MTP verify mask takes the tree path (per-token words equal to the common MTP mask's
  rows); clearing one prefix entry sends the batch to the general path.
* General masks (random, ragged query lengths up to 64, fully hidden rows, hidden prefix
  tokens, split requests, pages of 16 and 8, both 16-bit types) are checked with the
  north-star bound plus the normalised bounds and lse, after guards show that the check
  rejects the mask dropped, the mask shifted by one column and zeros on the same inputs.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import _lib
from batchspec_amd import masks as M
from batchspec_amd.workloads import make_verify_batch
from oracle import attention as OA
from tests import attn_parity as AP

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def oracle(b, mask):
    return OA.verify_attention(b.q.float().cpu().numpy(), b.cache.float().cpu().numpy(),
                               b.qo_indptr.cpu().numpy(), b.kv_indptr.cpu().numpy(),
                               b.kv_indices.cpu().numpy(), b.kv_last_page_len.cpu().numpy(),
                               b.page_size, mode="custom", custom_mask=mask, return_lse=True)


def plan_run(b, mask, **kw):
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(
        torch.empty(256 << 20, dtype=torch.uint8, device=DEV), "NHD", **kw)
    w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, b.num_qo_heads,
           b.num_kv_heads, b.head_dim, b.page_size, causal=False, q_data_type=b.q.dtype,
           custom_mask=mask)
    out, lse = w.run(b.q, b.cache, return_lse=True)
    torch.cuda.synchronize()
    return out, lse, w


def test_packing_matches_numpy():
    say("packbits, tree words and verdicts against numpy")
    rng = np.random.default_rng(5)
    # requests: (qo_len, kv_len, tree form?)
    shape = [(5, 40, True), (3, 3, True), (0, 17, True), (33, 50, False), (7, 70, False),
             (32, 32, True)]
    parts, qo_start, off, req = [], 0, 0, []
    for q, k, tree in shape:
        m = rng.random((q, k)) < 0.5
        if tree:
            m[:, : k - q] = True
        elif q <= 32:
            m[rng.integers(q), rng.integers(k - q)] = False  # a hidden prefix entry
        parts.append(m.ravel())
        req.append((qo_start, q, k, off))
        qo_start += q
        off += q * k
    req.append((qo_start, 2, 10, off))  # malformed: lies past the mask's end
    flat = np.concatenate(parts)
    n = flat.size
    # an unaligned device view: the byte-wise packing path
    store = torch.zeros(n + 1, dtype=torch.bool, device=DEV)
    store[1:] = torch.from_numpy(flat).to(DEV)
    mask_d = store[1:]
    B = len(req)
    req_d = torch.tensor(req, dtype=torch.int32, device=DEV)
    nw = (n + 31) // 32
    desc = torch.full((B + nw + 1,), -1, dtype=torch.int32, device=DEV)
    tree = torch.full((qo_start + 2,), -7, dtype=torch.int32, device=DEV)
    gen = torch.full((B,), -1, dtype=torch.int32, device=DEV)
    rc = _lib.load().bsx_custom_mask_prepare(mask_d.data_ptr(), n, req_d.data_ptr(), B,
                                            desc.data_ptr(), tree.data_ptr(), gen.data_ptr(),
                                            None)
    _lib.check(rc, "bsx_custom_mask_prepare")
    torch.cuda.synchronize()
    d = desc.cpu().numpy().view(np.uint32)
    want_bits = np.packbits(np.concatenate([flat, np.zeros(32 * nw - n, bool)]),
                            bitorder="little").view("<u4")
    np.testing.assert_array_equal(d[B:B + nw], want_bits)
    assert d[B + nw] == 0
    np.testing.assert_array_equal(d[:B], [r[3] for r in req])
    assert gen.cpu().tolist() == [0, 0, 0, 1, 1, 0, 2]
    t = tree.cpu().numpy().view(np.uint32)
    for (q0, q, k, o), (_, _, tr) in zip(req, shape):
        if not tr or q == 0:
            continue
        m = flat[o: o + q * k].reshape(q, k)[:, k - q:]
        want = (m.astype(np.uint64) << np.arange(q, dtype=np.uint64)).sum(1).astype(np.uint32)
        np.testing.assert_array_equal(t[q0: q0 + q], want)


def test_mtp_mask_takes_the_tree_path():
    say("MTP verify mask: device-packed tree words; one hidden prefix entry -> general")
    k = 4
    S = (k + 1) ** 2
    b = make_verify_batch(4, 20, 400, S, 32, 8, 128, 16, dtype=torch.bfloat16, seed=31).to(DEV)
    flat = M.mtp_verify_custom_mask(b.ctx.tolist(), k, device=DEV)
    out, lse, w = plan_run(b, flat)
    assert w.plan_info.mask_mode == _lib.MASK_TREE
    common, _ = M.mtp_attn_mask_and_position_ids(k)
    words = w._mask_words[: 4 * S].cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(words, np.tile(M.mask_to_words(common), 4))
    ref = oracle(b, flat.cpu().numpy())
    AP.check(out, ref[0], lse, ref[1])

    bad = flat.clone()
    bad[3] = False  # request 0, row 0 hides prefix token 3
    out2, lse2, w2 = plan_run(b, bad)
    assert w2.plan_info.mask_mode == _lib.MASK_CUSTOM
    assert w2.plan_info.shared_kv_tiles == 0
    ref2 = oracle(b, bad.cpu().numpy())
    AP.check(out2, ref2[0], lse2, ref2[1])
    assert not np.allclose(ref2[0][0], ref[0][0], atol=1e-3)  # the hidden token matters


def _general_mask(qo, kv, rng):
    parts = []
    for r, (q, k) in enumerate(zip(qo, kv)):
        m = rng.random((q, k)) < 0.55
        if q > 0 and r % 3 == 0:
            m[q // 2, :] = False  # a row that sees nothing: zeros, lse -inf
        if q > 1 and r % 3 == 1:
            m[:, : max(k - q, 1)] = True  # tree-like prefix, general tail
        parts.append(m.ravel())
    return np.concatenate(parts)


@pytest.mark.parametrize("dtype,ps,hq,hkv", [(torch.bfloat16, 16, 32, 8),
                                             (torch.float16, 8, 8, 8),
                                             (torch.bfloat16, 16, 28, 4)])
def test_general_masks_against_oracle(dtype, ps, hq, hkv):
    say(f"general custom masks: {dtype} page {ps} H={hq}/{hkv}")
    rng = np.random.default_rng(hq + ps)
    qo = np.array([1, 5, 33, 40, 17, 0, 64, 3])
    ctx = np.array([30, 200, 0, 90, 2500, 40, 100, 6000])
    b = make_verify_batch(8, 0, 0, 0, hq, hkv, 128, ps, dtype=dtype, scale=1.0, seed=hq + ps,
                          qo_lens=qo, ctx=ctx, device=DEV)
    kv = b.kv_lens
    mask = _general_mask(qo, kv, rng)
    out, lse, w = plan_run(b, torch.from_numpy(mask).to(DEV))
    assert w.plan_info.mask_mode == _lib.MASK_CUSTOM
    assert w.plan_info.num_split_requests > 0
    ref = oracle(b, mask)
    # guards: on these inputs the check tells the mask dropped, shifted by one column
    # and zeros apart from the reference
    shifted = np.concatenate([np.roll(p, 1) for p in np.split(mask, np.cumsum(qo * kv)[:-1])])
    AP.assert_discriminates(ref, [
        ("no mask", torch.from_numpy(oracle(b, np.ones_like(mask))[0]), None),
        ("shifted", torch.from_numpy(oracle(b, shifted)[0]), None),
        ("zeros", torch.zeros_like(out), None)])
    e, m = AP.check(out, ref[0], lse, ref[1])
    say(f"  max err {e:.3g} (max |ref| {m:.3g})")
    # the hidden rows: zeros and -inf
    assert torch.isinf(lse).any()


def test_graph_mode_refuses_general_masks():
    b = make_verify_batch(2, 40, 60, 5, 32, 8, 128, 16, dtype=torch.bfloat16, seed=3).to(DEV)
    mask = torch.ones(int(np.sum(5 * b.kv_lens)), dtype=torch.bool, device=DEV)
    mask[0] = False
    w = bsx.BatchPrefillWithPagedKVCacheWrapper(
        torch.empty(64 << 20, dtype=torch.uint8, device=DEV), "NHD", use_cuda_graph=True,
        qo_indptr_buf=b.qo_indptr.clone(), paged_kv_indptr_buf=b.kv_indptr.clone(),
        paged_kv_indices_buf=b.kv_indices.clone(),
        paged_kv_last_page_len_buf=b.kv_last_page_len.clone())
    with pytest.raises(NotImplementedError):
        w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, 32, 8, 128, 16,
               causal=False, q_data_type=torch.bfloat16, custom_mask=mask)
