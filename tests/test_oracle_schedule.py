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
    # the same workgroup shape as a host plan whose longest request has max_qo tokens (on
    # more than twice as many compute units as (request, kv head) pairs: the host-only
    # wave-split kernel, which a device plan never takes, needs at least half the units
    # in pairs; the shape compared does not depend on the unit count)
    qo = np.arange(B + 1, dtype=np.int32) * max_qo
    kvp = np.arange(B + 1, dtype=np.int32) * 4
    last = np.full(B, 16, np.int32)
    cus = 2 * B * hkv + 1
    bound = int(lib.bsx_attn_plan_ints_bound(B, cus))
    blob = np.empty(bound, np.int32)
    hp = _lib.AttnPlan()
    rc = lib.bsx_attn_plan(qo.ctypes.data, kvp.ctypes.data, last.ctypes.data, B, hq, hkv, d, 16,
                           mode, 64 if mode == 3 else 0, 512 if mode == 3 else 0, 0.0, cus, -1,
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
    assert lib.bsx_attn_plan_device(ctypes.byref(plan), p, p, p, -1, p, None) == -1
    rc = lib.bsx_attn_plan_device_shape(4, 32, 8, 128, 16, 1, 0, 0, 0.0, 256, 5, ctypes.byref(plan))
    assert rc == 0
    # null device pointers are refused
    assert lib.bsx_attn_plan_device(ctypes.byref(plan), None, p, p, -1, p, None) == -1
    assert lib.bsx_attn_plan_device(ctypes.byref(plan), p, p, p, -1, None, None) == -1


def _fixed_plan(lib, shape, qo, kvp, last, nidx=-1):
    qo, kvp, last = (np.ascontiguousarray(a, dtype=np.int32) for a in (qo, kvp, last))
    blob = np.full(int(shape.plan_ints), -7, np.int32)
    plan = _lib.AttnPlan()
    rc = lib.bsx_attn_plan_fixed(ctypes.byref(shape), qo.ctypes.data, kvp.ctypes.data,
                                 last.ctypes.data, len(qo) - 1, nidx, blob.ctypes.data,
                                 int(shape.plan_ints), ctypes.byref(plan))
    return rc, plan, blob


@pytest.mark.parametrize("mode,max_qo", [(1, 5), (2, 32), (3, 1)])
def test_fixed_layout_host_plan_keeps_every_launch_argument(mode, max_qo):
    """Graph mode: host plans of changing lengths (and fewer requests) laid out in one
    bound-sized shape keep every launch argument of bsx_attn_run, and each blob is a
    valid schedule (every tile once, slots and merge records consistent)."""
    lib = _lib.load()
    sink, window = (64, 512) if mode == 3 else (0, 0)
    shape = _lib.AttnPlan()
    assert lib.bsx_attn_plan_device_shape(64, 32, 8, 128, 16, mode, sink, window, 0.0, 256,
                                          max_qo, ctypes.byref(shape)) == 0
    skip = ("total_qo", "total_tiles")
    rng = np.random.default_rng(mode)
    for it in range(12):
        B = int(rng.integers(1, 65))
        qo_l = rng.integers(0 if it % 3 == 0 else 1, max_qo + 1, B)
        ctx = rng.integers(0, 9000 if mode != 3 else 70000, B)
        kv = ctx + qo_l
        pages = np.maximum(1, (kv + 15) // 16)
        last = np.where(kv > 0, (kv - 1) % 16 + 1, 0)
        kvp = np.concatenate([[0], np.cumsum(pages)])
        qo = np.concatenate([[0], np.cumsum(qo_l)])
        rc, plan, blob = _fixed_plan(lib, shape, qo, kvp, last, int(kvp[-1]))
        assert rc == 0, lib.bsx_last_error()
        for name, _ in shape._fields_:
            if name not in skip:
                assert getattr(plan, name) == getattr(shape, name), name
        assert plan.total_qo == qo[-1]
        s = OS.read_blob(blob, shape.batch, shape.num_ctas)
        assert s["dyn"][1] == 0
        OS.check_invariants(s, qo, kvp, last, 16, mode, sink, window)
        # requests past B are empty records that no segment names
        assert (s["seq"][B:, 1] == 0).all() and (s["seq"][B:, 2] == 0).all()
        assert (s["segments"][:, 0] < B).all()
        assert int(s["dyn"][2]) <= shape.num_segments
        # merge records fit their region (one per request), partial slots their bound
        assert int(s["dyn"][0]) <= shape.batch
        assert shape.off_merge_seqs + 4 * int(s["dyn"][0]) <= shape.off_part_indptr
        assert int(s["part"][-1]) <= shape.num_partials


def test_fixed_layout_host_plan_rejects():
    lib = _lib.load()
    shape = _lib.AttnPlan()
    assert lib.bsx_attn_plan_device_shape(4, 32, 8, 128, 16, 1, 0, 0, 0.0, 256, 5,
                                          ctypes.byref(shape)) == 0
    qo, kvp, last = [0, 5, 10], [0, 3, 9], [16, 4]
    assert _fixed_plan(lib, shape, qo, kvp, last, 9)[0] == 0
    # more query tokens than the fixed shape allows
    assert _fixed_plan(lib, shape, [0, 6, 11], kvp, last, 9)[0] == _lib.BSX_ERR_CAPACITY
    # the page table points past the kv_indices tensor
    assert _fixed_plan(lib, shape, qo, kvp, last, 8)[0] == _lib.BSX_ERR_INVALID
    # more requests than the shape
    assert _fixed_plan(lib, shape, [0, 1, 2, 3, 4, 5], [0, 1, 2, 3, 4, 5], [1] * 5)[0] != 0
    # a table without any page (run() has nothing to read)
    assert _fixed_plan(lib, shape, [0, 1, 2], [0, 0, 0], [0, 0])[0] == _lib.BSX_ERR_INVALID
    # a compact host plan refuses the same overflowing table
    bound = int(lib.bsx_attn_plan_ints_bound(2, 256))
    blob = np.empty(bound, np.int32)
    a = [np.ascontiguousarray(x, dtype=np.int32) for x in (qo, kvp, last)]
    rc = lib.bsx_attn_plan(a[0].ctypes.data, a[1].ctypes.data, a[2].ctypes.data, 2, 32, 8, 128, 16,
                           1, 0, 0, 0.0, 256, 8, blob.ctypes.data, bound,
                           ctypes.byref(_lib.AttnPlan()))
    assert rc == _lib.BSX_ERR_INVALID and b"exceeds" in lib.bsx_last_error()


def test_device_schedule_oracle_flags_an_overflowing_table():
    """The restatement of the device planner rejects kv_indptr[B] beyond the entries of
    kv_indices with an empty schedule, as the kernel does."""
    s = OS.schedule([0, 5, 10], [0, 3, 9], [16, 4], 16, 1, 0, 0, 5, 8, kv_indices_len=8)
    assert s["dyn"][1] == OS.ERR_INVALID and len(s["segments"]) == 0
    s = OS.schedule([0, 5, 10], [0, 3, 9], [16, 4], 16, 1, 0, 0, 5, 8, kv_indices_len=9)
    assert s["dyn"][1] == 0 and len(s["segments"]) > 0
