"""GPU parity of the device tree-mask producer (bsx_tree_masks) against the oracle's
ancestor mask, and end to end through verify attention: words built on the device give
bit-identical attention to the reference-style concatenated bool mask
(mtp_engine.py:410-417).  Bar: bit-exact."""
import sys

import numpy as np
import pytest
import torch

from batchspec_amd import masks as M
from batchspec_amd.workloads import make_verify_batch, random_tree_parents
from oracle import masks as OM

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _oracle_words(par):
    m, depth = OM.tree_ancestor_mask(par)
    n = len(par)
    w = (m.astype(np.uint64) << np.arange(n, dtype=np.uint64)).sum(1).astype(np.uint32)
    return w.view(np.int32), depth


def test_random_trees_per_request():
    say("tree masks: 40 random 32-node trees, per-request parents")
    rng = np.random.default_rng(5)
    B, n = 40, 32
    par = np.stack([random_tree_parents(n, rng) for _ in range(B)]).astype(np.int32)
    cl = rng.integers(0, 5000, B).astype(np.int32)
    words, pos = M.tree_masks(torch.from_numpy(par).to(DEV), torch.from_numpy(cl).to(DEV))
    for b in range(B):
        w, d = _oracle_words(par[b])
        np.testing.assert_array_equal(words[b].cpu().numpy(), w)
        np.testing.assert_array_equal(pos[b].cpu().numpy(), cl[b] + d)


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_mtp_layout_shared_parents(k):
    say(f"tree masks: MTP layout k={k}, shared parents")
    cl = torch.tensor([0, 17, 4000], dtype=torch.int32, device=DEV)
    par = torch.from_numpy(M.mtp_parents(k)).to(DEV)
    words, pos = M.tree_masks(par, cl)
    rm, rpos = OM.mtp_mask(k)
    S = rm.shape[0]
    rw = (rm.astype(np.uint64) << np.arange(S, dtype=np.uint64)).sum(1).astype(np.uint32).view(np.int32)
    for b in range(3):
        np.testing.assert_array_equal(words[b].cpu().numpy(), rw)
        np.testing.assert_array_equal(pos[b].cpu().numpy(), int(cl[b]) + rpos)


def test_parents_that_do_not_precede_end_the_chain():
    say("tree masks: invalid parents end the chain")
    par = torch.tensor([[-1, 0, 5, 2, -7, 3]], dtype=torch.int32, device=DEV)
    words, pos = M.tree_masks(par)
    # node 2's parent 5 does not precede it, node 4's is < -1: both are roots
    np.testing.assert_array_equal(words[0].cpu().numpy(), [1, 3, 4, 12, 16, 44])
    np.testing.assert_array_equal(pos[0].cpu().numpy(), [0, 1, 0, 1, 0, 2])


def test_device_words_drive_attention_like_the_bool_mask():
    say("MTP verify attention: device tree words vs reference bool mask (bitwise)")
    from batchspec_amd import BatchPrefillWithPagedKVCacheWrapper
    k = 4
    S = (k + 1) ** 2
    b = make_verify_batch(5, 20, 600, S, 32, 8, 128, 16, dtype=torch.bfloat16, seed=61).to(DEV)
    ctx = torch.as_tensor(b.ctx, dtype=torch.int32, device=DEV)
    outs = []
    for use_words in (False, True):
        w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(64 << 20, dtype=torch.uint8, device=DEV), "NHD")
        kw = {}
        if use_words:
            words, _ = M.tree_masks(torch.from_numpy(M.mtp_parents(k)).to(DEV), ctx)
            kw["tree_mask_words"] = words.flatten()
        else:
            kw["custom_mask"] = M.mtp_verify_custom_mask(b.ctx.tolist(), k, device=DEV)
        w.plan(b.qo_indptr, b.kv_indptr, b.kv_indices, b.kv_last_page_len, 32, 8, 128, 16,
               q_data_type=torch.bfloat16, causal=False, **kw)
        outs.append(w.run(b.q, b.cache))
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
