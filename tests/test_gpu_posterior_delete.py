"""The greedy acceptance fused with the delete of rejected tokens
(bsx_accept_greedy_delete through evaluate_posterior_and_delete) against the two calls it
replaces: evaluate_posterior (greedy branch of mtp_engine.py:553-560) followed by
DevicePageTable.delete_kv(n_inserted - accept_nums) (page_table.py:95-137).  Outputs
(bonus, accept, eos) and the whole page-table state must be equal bit for bit, and the
outputs must equal the oracle's greedy posterior; over logits and ids, both accept
rules, batches that take one and several rounds of the packed evaluation, and k = 0."""
import sys

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd.page_table import DevicePageTable
from batchspec_amd.workloads import greedy_case
from oracle import accept as OAc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PS = 16


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _table(B, ctx, n_inserted, max_pages):
    pt = DevicePageTable(PS, B, max_pages, DEV)
    pt.insert_kv(torch.from_numpy(ctx.astype(np.int32)).to(DEV))
    pt.insert_kv(n_inserted)
    return pt


def _state(pt):
    n = int(pt.paged_kv_indptr[-1])
    return [pt.cachelens.clone(), pt.paged_kv_indptr.clone(), pt.paged_kv_last_page_len.clone(),
            pt.page_manager.num_allocated_pages.clone(), pt.paged_kv_indices[:n].clone()]


@pytest.mark.parametrize("B,k,V,dt,rule,use_ids", [
    (64, 4, 128256, torch.bfloat16, "reference", False),
    (64, 4, 128256, torch.bfloat16, "prefix", False),
    (300, 7, 3000, torch.bfloat16, "reference", False),
    (5, 2, 1000, torch.float32, "prefix", False),
    (37, 0, 500, torch.float16, "reference", False),
    (130, 4, 2000, torch.float32, "reference", True),
    (9, 63, 256, torch.float32, "prefix", False),
])
def test_fused_acceptance_and_delete_equal_the_two_calls(B, k, V, dt, rule, use_ids):
    say(f"fused greedy acceptance + delete: B={B} k={k} V={V} {dt} rule={rule} ids={use_ids}")
    c = greedy_case(B=B, k=k, V=V, seed=B + k, dtype=dt)
    draft = c.draft_tokens.to(DEV)
    logits = c.target_logits.to(DEV)
    ids = torch.from_numpy(OAc.argmax(c.target_logits.float().numpy())).to(DEV)
    preds = ids if use_ids else logits
    eos = int(c.draft_tokens[0, 0]) if k > 0 else -1
    rng = np.random.default_rng(B)
    ctx = rng.integers(0, 700, B)
    n_ins = (k + 1) * (2 if B % 2 else 1)
    max_pages = (700 + n_ins) // PS + 3
    pt_f = _table(B, ctx, n_ins, max_pages)
    pt_r = _table(B, ctx, n_ins, max_pages)
    got = bsx.evaluate_posterior_and_delete(draft, preds, pt_f, n_ins, eos_token_id=eos,
                                            accept_rule=rule)
    want = bsx.evaluate_posterior(draft, preds, greedy=True, eos_token_id=eos, accept_rule=rule)
    pt_r.delete_kv((n_ins - want[1]).to(torch.int32))
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        assert g.dtype == w.dtype and torch.equal(g, w)
    for g, w in zip(_state(pt_f), _state(pt_r)):
        assert torch.equal(g, w)
    ref = OAc.greedy_posterior(c.draft_tokens.numpy(), c.target_logits.float().numpy(), eos, rule)
    np.testing.assert_array_equal(got[0].cpu().numpy()[:, 0], ref[0][:, 0])
    np.testing.assert_array_equal(got[1].cpu().numpy(), ref[1])
    np.testing.assert_array_equal(got[2].cpu().numpy()[:, 0], ref[2][:, 0])
    cl = pt_f.cachelens.cpu().numpy()
    # the step inserted n_ins tokens and deleted n_ins - accept: accept tokens remain
    np.testing.assert_array_equal(cl, ctx + ref[1])


def test_fused_acceptance_and_delete_refuse_bad_arguments():
    c = greedy_case(B=4, k=3, V=100, seed=1)
    pt = _table(4, np.full(4, 50), 4, 10)
    with pytest.raises(ValueError):  # deletes would be negative: n_inserted < k + 1
        bsx.evaluate_posterior_and_delete(c.draft_tokens.to(DEV), c.target_logits.to(DEV), pt, 3,
                                          eos_token_id=-1)
    with pytest.raises(ValueError):  # table of another batch
        bsx.evaluate_posterior_and_delete(c.draft_tokens[:3].to(DEV),
                                          c.target_logits[:3].to(DEV), pt, 4, eos_token_id=-1)
