"""gfx950 accepted-KV compaction (through the C ABI) against the oracle: bit-exact."""
import sys

import numpy as np
import pytest
import torch

from batchspec_amd.collate import collate_accepted_kv_cache
from oracle import collate as OC

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("dtype,k,ps,H,D", [(torch.bfloat16, 4, 16, 8, 128), (torch.float32, 3, 8, 2, 64),
                                            (torch.float16, 1, 1, 4, 64)])
def test_collate_bit_exact_multilayer(dtype, k, ps, H, D):
    say(f"collate dtype={dtype} k={k} ps={ps} H={H} D={D}")
    rng = np.random.default_rng(k * 100 + ps)
    B, ppr, L = 12, max(2, (k + 1) ** 2 // ps + 3), 3
    P = B * ppr + 5
    idx = rng.permutation(P)[: B * ppr].astype(np.int32)
    indptr = (np.arange(B + 1) * ppr).astype(np.int32)
    prev = rng.integers(0, ppr * ps - (k + 1) ** 2 + 1, size=B).astype(np.int32)
    acc = rng.integers(1, k + 2, size=B).astype(np.int64)
    acc[0], acc[1] = 1, k + 1
    caches = [torch.randn((P, 2, ps, H, D), dtype=torch.float32).to(dtype).to(DEV) for _ in range(L)]
    refs = [OC.collate(c.float().cpu().numpy(), acc, prev, k, indptr, idx, ps) for c in caches]
    collate_accepted_kv_cache(torch.from_numpy(acc).to(DEV), torch.from_numpy(prev).to(DEV), k, caches,
                              torch.from_numpy(indptr).to(DEV), torch.from_numpy(idx).to(DEV))
    torch.cuda.synchronize()
    for c, r in zip(caches, refs):
        np.testing.assert_array_equal(c.float().cpu().numpy(), r)


def test_collate_clamps_accept_and_stays_in_pages():
    say("collate: out-of-range accept counts")
    k, ps, H, D, B, ppr = 2, 4, 2, 64, 3, 3
    P = B * ppr
    idx = np.arange(P, dtype=np.int32)[::-1].copy()
    indptr = (np.arange(B + 1) * ppr).astype(np.int32)
    prev = np.array([0, 2, 8], np.int32)          # request 2: source 14 lies past its 12 slots
    acc = np.array([9, -3, 3], np.int64)          # clamped to [0, k+1]
    cache = torch.randn((P, 2, ps, H, D)).to(torch.bfloat16).to(DEV)
    before = cache.float().cpu().numpy()
    collate_accepted_kv_cache(torch.from_numpy(acc).to(DEV), torch.from_numpy(prev).to(DEV), k, cache,
                              torch.from_numpy(indptr).to(DEV), torch.from_numpy(idx).to(DEV))
    torch.cuda.synchronize()
    after = cache.float().cpu().numpy()
    # request 0: accept clamped to 3 -> positions 1, 2 take 3, 6
    lg = lambda a, b, p: a[idx[indptr[b] + p // ps], :, p % ps]
    np.testing.assert_array_equal(lg(after, 0, 1), lg(before, 0, 3))
    np.testing.assert_array_equal(lg(after, 0, 2), lg(before, 0, 6))
    # request 1: accept clamped to 0 -> untouched
    for p in range(ppr * ps):
        np.testing.assert_array_equal(lg(after, 1, p), lg(before, 1, p))
    # request 2: prev 8 -> source 11 moves to 9; source 14 is beyond the pages: skipped
    np.testing.assert_array_equal(lg(after, 2, 9), lg(before, 2, 11))
    for p in [q for q in range(ppr * ps) if q != 9]:
        np.testing.assert_array_equal(lg(after, 2, p), lg(before, 2, p))
