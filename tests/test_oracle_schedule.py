"""CPU checks of the device-side attention schedule: the restatement in
oracle/attn_schedule.py against the invariants every schedule must satisfy, and the
host-only bsx_attn_plan_device_shape against the restatement's layout."""
import ctypes

import numpy as np
import pytest

from batchspec_amd import _lib
from oracle import attn_schedule as OS


def random_table(rng, B, max_qo, page_size, max_ctx, empty_frac=0.2):
    qlen = rng.integers(1, max_qo + 1, B)
    qlen[rng.random(B) < empty_frac / 2] = 0
    ctx = rng.integers(0, max_ctx, B)
    kv = ctx + qlen
    kv[rng.random(B) < empty_frac / 2] = 0
    pages = np.maximum(1, (kv + page_size - 1) // page_size)
    last = np.where(kv > 0, (kv - 1) % page_size + 1, 0)
    return (np.concatenate([[0], np.cumsum(qlen)]), np.concatenate([[0], np.cumsum(pages)]), last)


@pytest.mark.parametrize("seed", range(12))
def test_schedule_restatement_invariants(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 90))
    ps = int(rng.choice([1, 16, 64]))
    mode = int(rng.choice([1, 2, 3]))
    sink, window = (64, 512) if mode == 3 else (0, 0)
    qo, kvp, last = random_table(rng, B, 8, ps, int(rng.choice([40, 3000, 70000])))
    W = int(rng.choice([1, 7, 64, 256]))
    s = OS.schedule(qo, kvp, last, ps, mode, sink, window, 8, W)
    assert s["dyn"][1] == 0
    OS.check_invariants(s, qo, kvp, last, ps, mode, sink, window)
    # shares are even: no workgroup's tiles exceed the mean share by more than a tile plus
    # the segment charges its share may hold
    segs, sp = s["segments"], s["seg_indptr"]
    loads = [int((segs[sp[w]:sp[w + 1], 2] - segs[sp[w]:sp[w + 1], 1]).sum()) for w in range(W)]
    total = sum(loads)
    assert max(loads) <= -(-total // max(1, min(W, total))) + 1 + 2 * 3


def test_schedule_errors():
    qo, kvp, last = np.array([0, 3, 12]), np.array([0, 2, 5]), np.array([16, 4])
    s = OS.schedule(qo, kvp, last, 16, 1, 0, 0, 8, 32)  # request 1 has 9 > 8 tokens
    assert s["dyn"][1] == OS.ERR_UNSUPPORTED and len(s["segments"]) == 0
    OS.check_invariants(s, qo, kvp, last, 16, 1, 0, 0)
    s = OS.schedule(qo, kvp, np.array([17, 4]), 16, 1, 0, 0, 9, 32)  # last page overfull
    assert s["dyn"][1] == OS.ERR_INVALID
    s = OS.schedule(np.array([0, 2]), np.array([0, 0]), np.array([0]), 16, 1, 0, 0, 4, 8)
    assert s["dyn"][1] == OS.ERR_INVALID  # no page in the table


@pytest.mark.parametrize("B,hq,hkv,d,max_qo,mode", [(64, 32, 8, 128, 5, 1), (32, 32, 8, 128, 32, 2),
                                                     (7, 28, 4, 128, 5, 1), (300, 8, 2, 64, 1, 3)])
def test_device_shape_layout(B, hq, hkv, d, max_qo, mode):
    lib = _lib.load()
    plan = _lib.AttnPlan()
    rc = lib.bsx_attn_plan_device_shape(B, hq, hkv, d, 16, mode, 64 if mode == 3 else 0,
                                        512 if mode == 3 else 0, 0.0, 256, max_qo,
                                        ctypes.byref(plan))
    assert rc == 0
    L = OS.layout(B, plan.num_ctas)
    assert plan.device_plan == 1 and plan.total_qo == B * max_qo
    assert (plan.off_seg_indptr, plan.off_segments, plan.off_merge_seqs, plan.off_part_indptr,
            plan.off_dyn, plan.plan_ints) == (L["off_seg_indptr"], L["off_segments"], L["off_merge"],
                                              L["off_part"], L["off_dyn"], L["ints"])
    assert plan.off_merge_seqs % 4 == 0 and plan.num_split_requests == B
    # the same workgroup shape as a host plan whose longest request has max_qo tokens
    qo = np.arange(B + 1, dtype=np.int32) * max_qo
    kvp = np.arange(B + 1, dtype=np.int32) * 4
    last = np.full(B, 16, np.int32)
    bound = int(lib.bsx_attn_plan_ints_bound(B, 256))
    blob = np.empty(bound, np.int32)
    hp = _lib.AttnPlan()
    rc = lib.bsx_attn_plan(qo.ctypes.data, kvp.ctypes.data, last.ctypes.data, B, hq, hkv, d, 16,
                           mode, 64 if mode == 3 else 0, 512 if mode == 3 else 0, 0.0, 256,
                           blob.ctypes.data, bound, ctypes.byref(hp))
    assert rc == 0
    for f in ("qrow_tile", "qrow_blocks", "heads_per_cta", "qblocks_per_cta", "num_qgroups",
              "shared_kv_tiles"):
        assert getattr(plan, f) == getattr(hp, f), f


def test_device_shape_rejects():
    lib = _lib.load()
    plan = _lib.AttnPlan()
    assert lib.bsx_attn_plan_device_shape(0, 32, 8, 128, 16, 1, 0, 0, 0.0, 256, 5,
                                          ctypes.byref(plan)) != 0
    assert lib.bsx_attn_plan_device_shape(4, 32, 8, 128, 16, 2, 0, 0, 0.0, 256, 33,
                                          ctypes.byref(plan)) != 0  # tree > 32 tokens
    assert lib.bsx_attn_plan_device_shape(5000, 32, 8, 128, 16, 1, 0, 0, 0.0, 256, 5,
                                          ctypes.byref(plan)) != 0  # batch above the bound


def test_device_plan_entry_rejects_bad_arguments():
    """bsx_attn_plan_device checks its arguments before launching anything (no GPU needed
    for these paths)."""
    lib = _lib.load()
    plan = _lib.AttnPlan()
    buf = np.zeros(16, np.int32)
    p = buf.ctypes.data
    # a host plan (device_plan == 0) is refused
    assert lib.bsx_attn_plan_device(ctypes.byref(plan), p, p, p, p, None) == -1
    rc = lib.bsx_attn_plan_device_shape(4, 32, 8, 128, 16, 1, 0, 0, 0.0, 256, 5, ctypes.byref(plan))
    assert rc == 0
    # null device pointers are refused
    assert lib.bsx_attn_plan_device(ctypes.byref(plan), None, p, p, p, None) == -1
    assert lib.bsx_attn_plan_device(ctypes.byref(plan), p, p, p, None, None) == -1
