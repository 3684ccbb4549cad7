"""GPU parity of the sync-free page-table update (DevicePageTable over
bsx_page_table_update) against the CPU restatement of PageTable.insert_kv / delete_kv
(batchspec/backends/base/page_table.py:55-137) and PageManager
(batchspec/backends/utils/paging.py:155-277): page counts, last-page lengths, the CSR
and cachelens bit-exact after every operation, including batches larger than one scan
chunk, refused over-allocations, and replays of a captured graph."""
import sys

import numpy as np
import pytest
import torch

from batchspec_amd.page_table import DevicePageTable
from oracle.paging import Pages

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class Ref:
    """oracle Pages plus cachelens (page_table.py:93,136)."""

    def __init__(self, B, P, ps):
        self.p = Pages(B, P, ps)
        self.p.allocate([1] * B)
        self.cl = np.zeros(B, np.int64)

    def apply(self, d, sign):
        d = [int(x) for x in d]
        if all(x <= 0 for x in d):
            return
        if sign > 0:
            self.p.insert_kv(d)  # raises before any change on over-allocation
        else:
            self.p.delete_kv(d)
        self.cl = np.maximum(self.cl + sign * np.asarray(d), 0)


def _check(t, ref):
    indptr, indices, last = ref.p.table()
    got_ptr = t.paged_kv_indptr.cpu().numpy()
    np.testing.assert_array_equal(got_ptr, indptr)
    np.testing.assert_array_equal(t.paged_kv_indices[: indptr[-1]].cpu().numpy(), indices)
    np.testing.assert_array_equal(t.paged_kv_last_page_len.cpu().numpy(), last)
    np.testing.assert_array_equal(t.page_manager.num_allocated_pages.cpu().numpy(), np.diff(indptr))
    np.testing.assert_array_equal(t.cachelens.cpu().numpy(), ref.cl)


@pytest.mark.parametrize("B,P,ps", [(64, 300, 16), (1500, 8, 4), (7, 40, 1), (9, 5, 64)])
def test_random_insert_delete_sequences(B, P, ps):
    say(f"page table: B={B} max_pages={P} page_size={ps}")
    rng = np.random.default_rng(B + P + ps)
    t = DevicePageTable(ps, B, P, DEV)
    ref = Ref(B, P, ps)
    _check(t, ref)
    for step in range(40):
        sign = 1 if rng.random() < 0.6 else -1
        if rng.random() < 0.3:
            d = int(rng.integers(-2, 2 * ps + 3))
            ds = [d] * B
            arg = d
        else:
            ds = rng.integers(-3, 2 * ps + 3, size=B)
            ds[rng.random(B) < 0.3] = 0
            arg = torch.from_numpy(ds.astype(np.int32)).to(DEV)
        try:
            ref.apply(ds, sign)
            refused = False
        except RuntimeError:
            refused = True
        (t.insert_kv if sign > 0 else t.delete_kv)(arg)
        if refused:
            with pytest.raises(RuntimeError):
                t.check()
        else:
            t.check()
        _check(t, ref)


def test_overallocation_is_refused_without_change():
    say("page table: refused insert leaves the state unchanged")
    t = DevicePageTable(16, 4, 3, DEV)
    ref = Ref(4, 3, 16)
    t.insert_kv(40)
    ref.apply([40] * 4, 1)
    _check(t, ref)
    d = torch.tensor([1, 0, 9, 0], dtype=torch.int32, device=DEV)  # request 2 would need 4 pages
    t.insert_kv(d)
    _check(t, ref)
    with pytest.raises(RuntimeError):
        t.check()
    t.check()  # counted once


def test_captured_graph_replays_match_eager():
    say("page table: insert/delete captured in a graph, replayed 3 times")
    B, P, ps = 64, 300, 16
    t = DevicePageTable(ps, B, P, DEV)
    ref = Ref(B, P, ps)
    rng = np.random.default_rng(9)
    acc = torch.from_numpy(rng.integers(1, 6, B).astype(np.int32)).to(DEV)
    acc_h = acc.cpu().numpy()
    t.insert_kv(100)
    ref.apply([100] * B, 1)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            t.insert_kv(25)       # a verify step's (k+1)^2 tokens
            t.delete_kv(25 - acc)  # keep the accepted ones
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    # capture recorded the work but did not run it
    _check(t, ref)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        ref.apply([25] * B, 1)
        ref.apply(25 - acc_h, -1)
        _check(t, ref)
