"""CPU tests of the drop-in boundary: the C-ABI library loads and exports every symbol
of include/bsx.h; the host planner's schedule is valid; the host-side mirrors
(page table, masks, custom-mask packing) match the oracle; the product refuses CPU
tensors instead of falling back."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import batchspec_amd as bsx
from batchspec_amd import _lib, masks
from oracle import masks as OM

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "bsx.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bsx_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_header_symbol(bsx):
    names = header_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(bsx, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes bindings must match the header"
    assert bsx.bsx_version() == 1


def test_rows_of_2_31_bytes_are_rejected_before_any_gpu_call():
    # the row statistics read logits through buffer descriptors (32-bit byte offsets):
    # every entry point that reaches them rejects a row of 2^31 bytes, before any HIP call
    L = _lib.load()
    unsupported = -3
    V32, V16 = 1 << 29, 1 << 30  # 2^31 bytes as fp32 / as 16-bit logits
    assert L.bsx_softmax(None, 2, 1.0, 1, V32, None, None, 0, None) == unsupported
    assert b"2^31 bytes" in L.bsx_last_error()
    assert L.bsx_softmax(None, 0, 1.0, 1, V16, None, None, 0, None) == unsupported
    assert L.bsx_softmax(None, 0, 1.0, 1, V16 - 1, None, None, 0, None) == -1  # null pointers
    assert L.bsx_chain_speculative_sampling_logits(None, None, None, 0, 1.0, None, 1, 1, V16,
                                                   None, None, None, None, 0, None) == unsupported
    assert L.bsx_chain_speculative_sampling_filtered(None, None, None, 0, 1.0, 20, 0.9, None, 1,
                                                     1, V16, None, None, None, None, 0,
                                                     None) == unsupported
    assert L.bsx_sampling_probs(None, 0, 1.0, 20, 0.9, 1, V16, None, None, 0,
                                None) == unsupported
    assert L.bsx_sample(None, 0, 1.0, 20, 0.9, None, 1, V16, None, None, 0, None) == unsupported


def _plan(qo, kvp, last, Hq=32, Hkv=8, D=128, ps=16, mode=_lib.MASK_CAUSAL, cus=256, sink=0,
          window=0, nidx=-1):
    L = _lib.load()
    qo, kvp, last = (np.ascontiguousarray(a, dtype=np.int32) for a in (qo, kvp, last))
    B = len(qo) - 1
    bound = L.bsx_attn_plan_ints_bound(B, cus)
    blob = np.zeros(bound, np.int32)
    plan = _lib.AttnPlan()
    rc = L.bsx_attn_plan(qo.ctypes.data, kvp.ctypes.data, last.ctypes.data, B, Hq, Hkv, D, ps, mode,
                         sink, window, 0.0, cus, nidx, blob.ctypes.data, bound,
                         ctypes.byref(plan))
    _lib.check(rc, "plan")
    return plan, blob


def _segments(plan, blob):
    segs = blob[plan.off_segments: plan.off_segments + 4 * plan.num_segments].reshape(-1, 4)
    indptr = blob[plan.off_seg_indptr: plan.off_seg_indptr + plan.num_ctas + 1]
    return segs, indptr


@pytest.mark.parametrize("cus", [1, 7, 256])
def test_plan_covers_every_tile_once_and_balances(cus):
    rng = np.random.default_rng(cus)
    B = 64
    ctx = rng.integers(1024, 4097, size=B)
    kv = ctx + 5
    pages = -(-kv // 16)
    kvp = np.concatenate([[0], np.cumsum(pages)])
    qo = np.arange(B + 1) * 5
    last = (kv - 1) % 16 + 1
    plan, blob = _plan(qo, kvp, last, cus=cus)
    segs, indptr = _segments(plan, blob)
    assert plan.heads_per_cta * plan.qblocks_per_cta <= 8
    assert np.all(np.diff(indptr) >= 0) and indptr[-1] == plan.num_segments
    covered = {b: np.zeros(-(-int(kv[b]) // 32), int) for b in range(B)}
    for b, t0, t1, slot in segs:
        covered[b][t0:t1] += 1
    assert all(np.all(c == 1) for c in covered.values())
    # balance: per workgroup cost = tiles + SEG_COST per segment (the planner's model);
    # the greedy packing loses less than one segment start per workgroup boundary
    SEG_COST = 2
    tiles = np.add.reduceat(segs[:, 2] - segs[:, 1], indptr[:-1])
    nseg = np.diff(indptr)
    cost = tiles + SEG_COST * nseg
    ideal = (np.sum(kv_tiles := -(-kv // 32)) + SEG_COST * B) / plan.num_ctas
    assert cost.max() <= np.ceil(ideal) + 2 * SEG_COST + 1, (cost.max(), ideal)
    assert plan.num_ctas <= cus * 2
    assert plan.total_tiles == int(np.sum(kv_tiles))
    # merge records (16-byte aligned): first slot, end slot, qo_start, qo_len per split request
    assert plan.off_merge_seqs % 4 == 0
    merge = blob[plan.off_merge_seqs: plan.off_merge_seqs + 4 * plan.num_split_requests].reshape(-1, 4)
    split = [b for b in range(B) if np.sum(segs[:, 0] == b) > 1]
    pip_ = blob[plan.off_part_indptr: plan.off_part_indptr + B + 1]
    assert merge[:, 0].tolist() == [int(pip_[b]) for b in split]
    assert merge[:, 1].tolist() == [int(pip_[b + 1]) for b in split]
    assert merge[:, 2].tolist() == [int(qo[b]) for b in split]
    assert merge[:, 3].tolist() == [int(qo[b + 1] - qo[b]) for b in split]
    # partial slots: contiguous per split request, unique
    slots = segs[segs[:, 3] >= 0, 3]
    assert len(set(slots.tolist())) == len(slots) == plan.num_partials
    pip = blob[plan.off_part_indptr: plan.off_part_indptr + B + 1]
    for b, t0, t1, slot in segs:
        if slot >= 0:
            assert pip[b] <= slot < pip[b + 1]
        else:
            assert pip[b] == pip[b + 1]


def test_plan_empty_kv_and_empty_queries():
    plan, blob = _plan([0, 3, 3, 5], [0, 1, 1, 2], [0, 0, 4])
    segs, _ = _segments(plan, blob)
    reqs = sorted(segs[:, 0].tolist())
    assert reqs == [0, 2]  # request 1 has no queries; request 0 (kv_len 0) still writes zeros
    assert all(s[1] == s[2] for s in segs if s[0] == 0)


def test_plan_streaming_skips_middle_tiles():
    kv = 5000
    plan, blob = _plan([0, 1], [0, -(-kv // 16)], [(kv - 1) % 16 + 1], mode=_lib.MASK_STREAMING,
                       sink=64, window=512, cus=4)
    segs, _ = _segments(plan, blob)
    tiles = sorted(t for s in segs for t in range(s[1], s[2]))
    assert tiles == list(range(0, 2)) + list(range((kv - 512) // 32, -(-kv // 32)))


def test_plan_custom_masks_cover_every_tile_on_the_per_wave_kernel():
    # 25 query tokens x group 4 = 100 rows: the tree mode takes the shared-tile kernel,
    # a general custom mask the per-wave one (it reads mask bits per row); every tile of
    # every request is scheduled either way, and the custom mode accepts qo_len > 32
    qo = np.array([0, 25, 50, 90])
    kv = np.array([300, 2000, 1000])
    kvp = np.concatenate([[0], np.cumsum(-(-kv // 16))])
    last = (kv - 1) % 16 + 1
    with pytest.raises(NotImplementedError, match="tree mask"):
        _plan(qo, kvp, last, mode=_lib.MASK_TREE)
    pt, _ = _plan(qo[:3], kvp[:3], last[:2], mode=_lib.MASK_TREE)
    assert pt.shared_kv_tiles == 1
    pc, blob = _plan(qo, kvp, last, mode=_lib.MASK_CUSTOM)
    assert pc.shared_kv_tiles == 0 and pc.mask_mode == _lib.MASK_CUSTOM
    segs, _ = _segments(pc, blob)
    for b in range(3):
        tiles = sorted(t for s in segs if s[0] == b for t in range(s[1], s[2]))
        assert tiles == list(range(-(-int(kv[b]) // 32)))
    with pytest.raises(ValueError, match="unknown mask mode"):
        _plan(qo, kvp, last, mode=5)


@pytest.mark.parametrize("bad,exc", [
    (dict(D=96), NotImplementedError),
    (dict(Hq=30, Hkv=8), ValueError),
    (dict(ps=12), NotImplementedError),
])
def test_plan_rejects_unsupported(bad, exc):
    with pytest.raises(exc):
        _plan([0, 5], [0, 1], [5], **bad)


def test_plan_rejects_bad_page_table():
    with pytest.raises(ValueError, match="last_page_len"):
        _plan([0, 5], [0, 1], [17])
    with pytest.raises(ValueError, match="non-decreasing"):
        _plan([0, 5, 4], [0, 1, 2], [3, 3])
    with pytest.raises(NotImplementedError, match="tree mask"):
        _plan([0, 33], [0, 3], [16], mode=_lib.MASK_TREE)


@pytest.mark.parametrize("k", [1, 2, 4])
def test_mtp_mask_mirror_matches_oracle(k):
    m, pos = masks.mtp_attn_mask_and_position_ids(k)
    rm, rpos = OM.mtp_mask(k)
    np.testing.assert_array_equal(m.numpy(), rm)
    np.testing.assert_array_equal(pos.numpy(), rpos)


def test_tree_words_match_oracle_ancestor_mask():
    from batchspec_amd.workloads import random_tree_parents
    rng = np.random.default_rng(3)
    for _ in range(20):
        par = random_tree_parents(32, rng)
        w, d = masks.tree_mask_words(par)
        m, depth = OM.tree_ancestor_mask(par)
        np.testing.assert_array_equal(masks.mask_to_words(torch.from_numpy(m)), w)
        np.testing.assert_array_equal(d, depth)
        assert depth.max() <= 6


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_mtp_parents_give_the_mtp_mask(k):
    # the MTP layout read as a tree: its ancestor relation and depths are the closed form
    # of mtp_engine.py:172-208 (pinned by the k = 2 known answer of mtp_engine.py:360-368)
    par = masks.mtp_parents(k)
    m, depth = OM.tree_ancestor_mask(par)
    rm, rpos = OM.mtp_mask(k)
    np.testing.assert_array_equal(m, rm)
    np.testing.assert_array_equal(depth, rpos)
    assert np.all(par < np.arange(par.size))


def test_product_has_no_cpu_path():
    x = torch.zeros(2, 8)
    with pytest.raises(ValueError, match="no CPU path"):
        bsx.sampling.argmax(x)
    with pytest.raises(ValueError, match="no CPU path"):
        bsx.get_seq_lens(torch.zeros(3, dtype=torch.int32), torch.zeros(2, dtype=torch.int32), 16)
    with pytest.raises(ValueError, match="no CPU path"):
        bsx.BatchPrefillWithPagedKVCacheWrapper(torch.empty(1024, dtype=torch.uint8))


def test_plan_wave_split_for_short_views_that_fill_the_device():
    """The host planner takes the wave-split kernel (shared_kv_tiles 2: one workgroup per
    request and kv head, no partials) when every view has at most 32 tiles, a kv head has
    at most 16 query rows, the (request, kv head) pairs number between half the compute
    units and all of them, and its time model puts it ahead of the split-KV schedule;
    any other shape keeps the split-KV schedule."""
    B = 32
    rng = np.random.default_rng(0)
    ctx = rng.integers(32768, 65536, B)
    pages = -(-(ctx + 1) // 16)
    kvp = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    last = ((ctx + 1 - 1) % 16 + 1).astype(np.int32)
    qo = np.arange(B + 1, dtype=np.int32)  # one query token each
    # config 3a: a 64-sink + 512-window view (19 tiles) of 32k-64k tokens, 32 x 8 pairs
    p, _ = _plan(qo, kvp, last, mode=_lib.MASK_STREAMING, sink=64, window=512)
    assert p.shared_kv_tiles == 2 and p.num_partials == 0 and p.num_split_requests == 0
    assert p.float_ws_bytes == 0 and p.num_ctas == B and p.heads_per_cta == 1
    # down to half the units (256 pairs on 512), then no further
    p, _ = _plan(qo, kvp, last, mode=_lib.MASK_STREAMING, sink=64, window=512, cus=512)
    assert p.shared_kv_tiles == 2
    p, _ = _plan(qo, kvp, last, mode=_lib.MASK_STREAMING, sink=64, window=512, cus=513)
    assert p.shared_kv_tiles != 2
    # more pairs than units: two workgroups per unit fall behind the balanced split
    p, _ = _plan(qo, kvp, last, mode=_lib.MASK_STREAMING, sink=64, window=512, cus=255)
    assert p.shared_kv_tiles != 2
    # the full causal view (1000+ tiles), 5 query tokens x 4 rows: split-KV
    p, _ = _plan(qo, kvp, last, mode=_lib.MASK_CAUSAL)
    assert p.shared_kv_tiles != 2
    qo5 = np.arange(B + 1, dtype=np.int32) * 5
    p, _ = _plan(qo5, kvp, last, mode=_lib.MASK_STREAMING, sink=64, window=512)
    assert p.shared_kv_tiles != 2
    # the time model: 16 single-token requests (128 pairs) of 32-tile views favour the
    # split (the longest view's run per wave, 4 tiles, against 2 MB per compute unit);
    # 4-token drafts over the same views (16 rows per kv head: partials to merge) and
    # 10-tile views favour the wave split
    def views(n, tiles, q):
        kv = np.full(n, 32 * tiles, np.int64)
        return (np.arange(n + 1, dtype=np.int32) * q,
                np.concatenate([[0], np.cumsum(kv // 16)]).astype(np.int32), np.full(n, 16, np.int32))
    p, _ = _plan(*views(16, 32, 1))
    assert p.shared_kv_tiles != 2
    p, _ = _plan(*views(16, 32, 4))
    assert p.shared_kv_tiles == 2
    p, _ = _plan(*views(16, 10, 1))
    assert p.shared_kv_tiles == 2
    # at head dim 64 a wave's tile takes half the time: the 32-tile single-token views go
    # to the wave split too (measured 13.9 against 16.9 us)
    p, _ = _plan(*views(16, 32, 1), D=64)
    assert p.shared_kv_tiles == 2
