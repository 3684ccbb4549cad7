"""Pins the attention oracle (oracle/attention.py) against independent references:
torch's scaled_dot_product_attention, pure-Python loops and exact invariances."""
import math

import numpy as np
import pytest
import torch

from batchspec_amd.workloads import make_verify_batch
from oracle import attention as OA
from oracle import masks as OM


def _np(b):
    return (b.q.float().numpy(), b.cache.float().numpy(), b.qo_indptr.numpy(),
            b.kv_indptr.numpy(), b.kv_indices.numpy(), b.kv_last_page_len.numpy())


def _sdpa_reference(b, vis_fn):
    """torch SDPA per request on contiguously gathered KV (GQA by repeat_interleave)."""
    q, cache, qo, kvp, idx, last = _np(b)
    lens = OA.seq_lens(kvp, last, b.page_size)
    g = b.num_qo_heads // b.num_kv_heads
    out = np.zeros_like(q)
    for r in range(len(qo) - 1):
        q0, q1 = qo[r], qo[r + 1]
        L = int(lens[r])
        pages = idx[kvp[r] + np.arange(L) // b.page_size]
        slots = np.arange(L) % b.page_size
        K = torch.from_numpy(cache[pages, 0, slots]).permute(1, 0, 2)  # [Hkv, L, D]
        V = torch.from_numpy(cache[pages, 1, slots]).permute(1, 0, 2)
        K = K.repeat_interleave(g, 0)
        V = V.repeat_interleave(g, 0)
        Q = torch.from_numpy(q[q0:q1]).permute(1, 0, 2)
        m = torch.from_numpy(vis_fn(q1 - q0, L, r))
        o = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=m)
        out[q0:q1] = o.permute(1, 0, 2).numpy()
    return out


@pytest.mark.parametrize("seed", [0, 1])
def test_causal_matches_torch_sdpa(seed):
    b = make_verify_batch(3, 20, 70, 5, 8, 2, 64, 16, dtype=torch.float32, seed=seed)
    got = OA.verify_attention(*_np(b), b.page_size, mode="causal")
    ref = _sdpa_reference(b, lambda q, L, r: OA.visibility("causal", q, L))
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)


def test_custom_mask_matches_torch_sdpa():
    b = make_verify_batch(2, 30, 40, 6, 4, 4, 64, 8, dtype=torch.float32, seed=3)
    rng = np.random.default_rng(0)
    lens = b.kv_lens
    masks = [rng.random((6, int(L))) < 0.6 for L in lens]
    for m in masks:
        m[:, 0] = True  # every row sees something
    flat = np.concatenate([m.ravel() for m in masks])
    got = OA.verify_attention(*_np(b), b.page_size, mode="custom", custom_mask=flat)
    ref = _sdpa_reference(b, lambda q, L, r: masks[r])
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)


def test_pure_python_loops_tiny():
    b = make_verify_batch(2, 3, 9, 2, 2, 1, 64, 4, dtype=torch.float32, seed=7)
    q, cache, qo, kvp, idx, last = _np(b)
    got = OA.verify_attention(q, cache, qo, kvp, idx, last, 4, mode="causal")
    lens = OA.seq_lens(kvp, last, 4)
    D = q.shape[2]
    for r in range(2):
        for t in range(qo[r + 1] - qo[r]):
            for h in range(2):
                L = int(lens[r])
                scores = []
                for j in range(L):
                    if j > L - (qo[r + 1] - qo[r]) + t:
                        continue
                    page = idx[kvp[r] + j // 4]
                    s = sum(float(q[qo[r] + t, h, d]) * float(cache[page, 0, j % 4, 0, d])
                            for d in range(D)) / math.sqrt(D)
                    scores.append((s, page, j % 4))
                mx = max(s for s, _, _ in scores)
                w = [math.exp(s - mx) for s, _, _ in scores]
                tot = sum(w)
                for d in range(0, D, 13):
                    o = sum(wi * float(cache[p, 1, sl, 0, d]) for wi, (_, p, sl) in zip(w, scores)) / tot
                    assert abs(o - got[qo[r] + t, h, d]) < 1e-5


def test_page_permutation_invariance():
    b = make_verify_batch(3, 40, 90, 5, 8, 2, 64, 16, dtype=torch.float32, seed=11)
    q, cache, qo, kvp, idx, last = _np(b)
    base = OA.verify_attention(q, cache, qo, kvp, idx, last, 16)
    perm = np.random.default_rng(1).permutation(cache.shape[0])
    new_cache = np.empty_like(cache)
    new_cache[perm] = cache           # physical page p moves to perm[p]
    new_idx = perm[idx].astype(np.int32)
    moved = OA.verify_attention(q, new_cache, qo, kvp, new_idx, last, 16)
    np.testing.assert_array_equal(base, moved)


def test_chain_tree_equals_causal_and_decode_equals_full():
    b = make_verify_batch(2, 30, 60, 5, 4, 2, 64, 16, dtype=torch.float32, seed=5)
    args = _np(b)
    causal = OA.verify_attention(*args, 16, mode="causal")
    lens = b.kv_lens
    chain = np.concatenate([OA.visibility("causal", 5, int(L)).ravel() for L in lens])
    tree = OA.verify_attention(*args, 16, mode="custom", custom_mask=chain)
    np.testing.assert_array_equal(causal, tree)
    d = make_verify_batch(3, 30, 60, 1, 4, 2, 64, 16, dtype=torch.float32, seed=6)
    np.testing.assert_array_equal(OA.verify_attention(*_np(d), 16, mode="causal"),
                                  OA.verify_attention(*_np(d), 16, mode="none"))


def test_gqa_equals_repeated_kv_heads():
    b = make_verify_batch(2, 20, 50, 3, 8, 2, 64, 16, dtype=torch.float32, seed=9)
    q, cache, qo, kvp, idx, last = _np(b)
    got = OA.verify_attention(q, cache, qo, kvp, idx, last, 16)
    mha = np.repeat(cache, 4, axis=3)  # kv head h//4 -> 8 heads
    ref = OA.verify_attention(q, mha, qo, kvp, idx, last, 16)
    np.testing.assert_allclose(got, ref, rtol=0, atol=0)


def test_streaming_view_equals_compacted_cache():
    sink, window = 8, 24
    b = make_verify_batch(2, 80, 120, 5, 4, 2, 64, 16, dtype=torch.float32, seed=12)
    q, cache, qo, kvp, idx, last = _np(b)
    got = OA.verify_attention(q, cache, qo, kvp, idx, last, 16, mode="streaming", sink=sink,
                              window=window)
    # compact each request's visible tokens into a fresh contiguous paged cache
    lens = OA.seq_lens(kvp, last, 16)
    for r in range(2):
        L = int(lens[r])
        keep = np.r_[0:sink, L - window:L]
        K, V = OA.gather_kv(cache, kvp, idx, 16, r, L)
        comp = np.zeros((len(keep), 2, 1, 2, 64), np.float32)
        comp[:, 0, 0], comp[:, 1, 0] = K[keep], V[keep]
        qq = q[qo[r]:qo[r + 1]]
        ref = OA.verify_attention(qq, comp, [0, 5], [0, len(keep)], np.arange(len(keep)),
                                  [1], 1, mode="causal")
        np.testing.assert_allclose(got[qo[r]:qo[r + 1]], ref, rtol=1e-6, atol=1e-6)


def test_masks_known_answer_k2():
    # batchspec/backends/mtp_engine.py:360-368
    expected = np.array([[1, 0, 0, 0, 0, 0], [1, 1, 0, 0, 0, 0], [1, 1, 1, 0, 0, 0],
                         [1, 0, 0, 1, 0, 0], [1, 0, 0, 1, 1, 0], [1, 0, 0, 1, 1, 1]], dtype=bool)
    m, pos = OM.mtp_mask(2)
    # the docstring shows the k=2 example over 6 tokens: the leading 6x6 block
    np.testing.assert_array_equal(m[:6, :6], expected)
    np.testing.assert_array_equal(pos[:6], [0, 1, 2, 1, 2, 3])
