"""Verify attention behind FlashInfer's ``BatchPrefillWithPagedKVCacheWrapper`` surface.

BatchSpec builds the wrapper at batchspec/backends/base/attn_wrapper.py:53-72
(NHD layout, ``use_cuda_graph=True``, fixed page-table buffers, optional custom-mask
buffers), plans it once per step (batchspec/backends/standard_engine.py:132-143,
batchspec/backends/mtp_engine.py:331-342,420-432,486-497) and runs it in every layer
(batchspec/models/modules/attention/standard.py:69).  This class keeps that
constructor, ``plan`` and ``run``; the compute is the gfx950 kernel of
``libbsx.so``.

Supported plan options: ``causal`` (bottom-right aligned); ``custom_mask``, any
flattened boolean mask of sum(qo_len * kv_len) entries, packed on the device (masks
whose prefix columns are all visible and whose last ``qo_len`` columns form an at most
32-wide block, the MTP and EAGLE-tree masks, take the fast tree path; others the general
one); the equivalent per-query-token ``tree_mask_words``; and a StreamingLLM sink +
window view (``sink_tokens``, ``window_tokens``) for MagicDec-style draft attention.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import _lib
from ._util import dtype_code, num_cus, require_gpu, stream_of

_ALIGN = 256


def _align(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def _host_i32(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().to("cpu", torch.int32).numpy())


class BatchPrefillWithPagedKVCacheWrapper:
    """Paged-KV attention for ragged batches of verify / prefill queries (gfx950)."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, qo_indptr_buf: Optional[torch.Tensor] = None,
                 paged_kv_indptr_buf: Optional[torch.Tensor] = None,
                 paged_kv_indices_buf: Optional[torch.Tensor] = None,
                 paged_kv_last_page_len_buf: Optional[torch.Tensor] = None,
                 custom_mask_buf: Optional[torch.Tensor] = None,
                 mask_indptr_buf: Optional[torch.Tensor] = None,
                 backend: str = "auto", **unused) -> None:
        if kv_layout != "NHD":
            raise NotImplementedError(f"kv_layout {kv_layout!r}: only 'NHD' is implemented")
        if backend not in ("auto", "bsx"):
            raise NotImplementedError(f"backend {backend!r}")
        self._device = require_gpu("workspace", float_workspace_buffer)
        _lib.load()
        self._ws = float_workspace_buffer.view(torch.uint8).reshape(-1)
        self._use_cuda_graph = bool(use_cuda_graph)
        self._qo_indptr_buf = qo_indptr_buf
        self._kv_indptr_buf = paged_kv_indptr_buf
        self._kv_indices_buf = paged_kv_indices_buf
        self._kv_last_buf = paged_kv_last_page_len_buf
        self._custom_mask_buf = custom_mask_buf
        self._mask_indptr_buf = mask_indptr_buf
        if self._use_cuda_graph and paged_kv_indices_buf is None:
            raise ValueError("use_cuda_graph=True needs paged_kv_indices_buf")
        self._num_cus = num_cus(self._device.index if self._device.index is not None
                                else torch.cuda.current_device())
        self._plan: Optional[_lib.AttnPlan] = None
        self._kv_indices: Optional[torch.Tensor] = None
        self._mask_words: Optional[torch.Tensor] = None
        self._custom_desc: Optional[torch.Tensor] = None  # packed general custom mask
        self._blob_bytes = 0
        self._pinned: Optional[torch.Tensor] = None
        self._pinned_tab: Optional[torch.Tensor] = None
        self._copy_done: Optional[torch.cuda.Event] = None
        self._dtype: Optional[torch.dtype] = None
        # device plans: the int32 page-table tensors the planner reads (kept alive while
        # a captured graph may replay them)
        self._dev_idx: list = []
        # graph mode: the fixed shape every host plan is laid out in, and the launch
        # arguments of the plan a captured run() replays (None until a capture)
        self._graph_shape: Optional[_lib.AttnPlan] = None
        self._graph_static: Optional[tuple] = None
        self._captured_sig: Optional[tuple] = None
        self._captured_rows = 0
        self._host_blob: Optional[np.ndarray] = None

    # ------------------------------------------------------------------ plan
    def plan(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor,
             paged_kv_indices: torch.Tensor, paged_kv_last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim_qk: int, page_size: int,
             head_dim_vo: Optional[int] = None, custom_mask: Optional[torch.Tensor] = None,
             packed_custom_mask: Optional[torch.Tensor] = None, causal: bool = False,
             pos_encoding_mode: str = "NONE", use_fp16_qk_reduction: bool = False,
             sm_scale: Optional[float] = None, window_left: int = -1,
             logits_soft_cap: Optional[float] = None, rope_scale: Optional[float] = None,
             rope_theta: Optional[float] = None, q_data_type: Union[str, torch.dtype] = "float16",
             kv_data_type: Union[str, torch.dtype, None] = None, non_blocking: bool = True,
             *, tree_mask_words: Optional[torch.Tensor] = None, sink_tokens: int = 0,
             window_tokens: int = 0, on_device: bool = False,
             max_qo_len: Optional[int] = None) -> None:
        """Schedule one step of attention; shared by every layer until the next plan.

        Mirrors FlashInfer's plan (arguments as passed at
        batchspec/backends/standard_engine.py:132-143).  Host-synchronising: the
        indptr arrays are read on the host, as FlashInfer does.

        With ``use_cuda_graph=True`` (how BatchSpec builds the wrapper,
        batchspec/backends/base/attn_wrapper.py:53-57) the schedule is written into a
        fixed, bound-sized layout (requests up to ``qo_indptr_buf``'s size, query tokens
        per request up to the largest seen, or ``max_qo_len`` when given), so a graph
        that captured run() replays every later plan of that shape.  A later plan that
        needs a larger shape raises ValueError once a graph has captured run().

        With ``on_device=True`` (no counterpart in the reference) the schedule is
        computed on the GPU from the device tensors, stream-ordered and without a host
        synchronisation, so plan() and run() can be captured in one graph and replayed
        with page-table lengths that change between replays.  ``max_qo_len`` bounds
        every request's query tokens; q and out then need ``batch * max_qo_len`` token
        rows.  Masks: causal, sink+window, or ``tree_mask_words`` (device tensor, one
        word per token row); a boolean ``custom_mask`` needs a host plan.
        Malformed tables are reported by :meth:`device_plan_error`, not raised.
        """
        if head_dim_vo is not None and head_dim_vo != head_dim_qk:
            raise NotImplementedError("head_dim_vo != head_dim_qk")
        if packed_custom_mask is not None:
            raise NotImplementedError("packed_custom_mask; pass custom_mask or tree_mask_words")
        if pos_encoding_mode != "NONE":
            raise NotImplementedError("RoPE is applied by the caller (pos_encoding_mode='NONE')")
        if logits_soft_cap not in (None, 0.0) or window_left not in (-1, None):
            raise NotImplementedError("logits_soft_cap / window_left")
        if use_fp16_qk_reduction:
            raise NotImplementedError("use_fp16_qk_reduction")
        qdt = _as_dtype(q_data_type)
        if qdt not in (torch.bfloat16, torch.float16):
            raise NotImplementedError(f"q_data_type {qdt}: bf16 and fp16 are implemented")
        kdt = _as_dtype(kv_data_type) if kv_data_type is not None else qdt
        if kdt != qdt:
            raise NotImplementedError("kv_data_type must equal q_data_type")

        if on_device:
            self._plan_on_device(qo_indptr, paged_kv_indptr, paged_kv_indices,
                                 paged_kv_last_page_len, num_qo_heads, num_kv_heads, head_dim_qk,
                                 page_size, custom_mask, causal, sm_scale, qdt, tree_mask_words,
                                 sink_tokens, window_tokens, max_qo_len, non_blocking)
            return

        qo_h, kvp_h, last_h = self._host_tables(qo_indptr, paged_kv_indptr,
                                                paged_kv_last_page_len)
        batch = int(qo_h.shape[0]) - 1
        if batch < 0 or kvp_h.shape[0] != batch + 1 or last_h.shape[0] < batch:
            raise ValueError("qo_indptr, paged_kv_indptr and paged_kv_last_page_len disagree on batch")
        last_h = np.ascontiguousarray(last_h[:batch])

        streaming = sink_tokens > 0 or window_tokens > 0
        words = None
        packed = None
        if tree_mask_words is not None or custom_mask is not None:
            if causal or streaming:
                raise ValueError("custom/tree mask cannot be combined with causal or streaming")
            mode = _lib.MASK_TREE
            if tree_mask_words is not None:
                words = tree_mask_words
            else:
                qo_lens = np.diff(qo_h)
                npages = np.diff(kvp_h)
                kv_lens = np.where(npages > 0, (npages - 1) * page_size + last_h, 0)
                packed = self._pack_custom_mask(custom_mask, qo_h, qo_lens, kv_lens)
                mode, words = packed[0], packed[2]
        elif streaming:
            mode = _lib.MASK_STREAMING
        elif causal:
            mode = _lib.MASK_CAUSAL
        else:
            mode = _lib.MASK_NONE

        lib = _lib.load()
        nidx = int(paged_kv_indices.numel())
        if int(kvp_h[-1]) > nidx:
            raise ValueError(f"paged_kv_indptr[-1] = {int(kvp_h[-1])} exceeds the {nidx} entries "
                             "of paged_kv_indices")
        plan = _lib.AttnPlan()
        if self._use_cuda_graph:
            # FlashInfer's graph mode: plan() may be called again with other lengths and a
            # graph that captured run() replays the new plan.  Every launch argument must
            # therefore stay fixed: the schedule is laid out in a bound-sized shape.
            static = (int(num_qo_heads), int(num_kv_heads), int(head_dim_qk), int(page_size),
                      mode, int(sink_tokens), int(window_tokens), float(sm_scale or 0.0))
            max_qo = int(np.diff(qo_h).max()) if batch > 0 else 0
            # the shape is adopted only once the plan passes _check_captured below
            shape = self._fixed_shape(lib, batch, max(max_qo, int(max_qo_len or 0)), static)
            new_shape = (shape, static)
            bound = int(shape.plan_ints)
            blob = np.zeros(bound, dtype=np.int32)
            rc = lib.bsx_attn_plan_fixed(ctypes.byref(shape), qo_h.ctypes.data, kvp_h.ctypes.data,
                                         last_h.ctypes.data, batch, nidx, blob.ctypes.data, bound,
                                         ctypes.byref(plan))
            _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.plan")
            blob_bytes = _align(bound * 4)
        else:
            new_shape = None
            bound = int(lib.bsx_attn_plan_ints_bound(batch, self._num_cus))
            blob = np.empty(bound, dtype=np.int32)
            rc = lib.bsx_attn_plan(qo_h.ctypes.data, kvp_h.ctypes.data, last_h.ctypes.data, batch,
                                   int(num_qo_heads), int(num_kv_heads), int(head_dim_qk),
                                   int(page_size), mode, int(sink_tokens), int(window_tokens),
                                   float(sm_scale) if sm_scale else 0.0, self._num_cus, nidx,
                                   blob.ctypes.data, bound, ctypes.byref(plan))
            _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.plan")
            blob_bytes = _align(bound * 4)
        need = blob_bytes + int(plan.float_ws_bytes)
        if need > self._ws.numel():
            raise ValueError(f"float_workspace_buffer too small: need {need} bytes, "
                             f"have {self._ws.numel()}")
        self._check_captured(plan, blob_bytes)
        if new_shape is not None:
            self._graph_shape, self._graph_static = new_shape
        self._blob_bytes = blob_bytes
        self._host_blob = blob[: int(plan.plan_ints)].copy()

        # Stage the blob through pinned memory; the previous copy must have landed
        # before its staging buffer is rewritten.
        n = int(plan.plan_ints)
        if self._pinned is None or self._pinned.numel() < bound:
            if self._copy_done is not None:
                self._copy_done.synchronize()
            self._pinned = torch.empty(bound, dtype=torch.int32, pin_memory=True)
        elif self._copy_done is not None:
            self._copy_done.synchronize()
        self._pinned[:n].copy_(torch.from_numpy(blob[:n]))
        dev_blob = self._ws[:n * 4].view(torch.int32)
        with torch.cuda.device(self._device):
            dev_blob.copy_(self._pinned[:n], non_blocking=True)
            if self._copy_done is None:
                self._copy_done = torch.cuda.Event()
            self._copy_done.record()

        self._set_kv_indices(paged_kv_indices, non_blocking)
        if words is not None:
            self._set_mask_words(words, int(plan.total_qo))
        if packed is not None:
            self._custom_desc = packed[1]
        self._plan = plan
        self._dtype = qdt

    def _pack_custom_mask(self, custom_mask: torch.Tensor, qo_h: np.ndarray, qo_lens: np.ndarray,
                          kv_lens: np.ndarray):
        """plan(custom_mask=...) as FlashInfer's plan() takes it (the MTP engine's call at
        batchspec/backends/mtp_engine.py:399-432): the flattened boolean mask of
        sum(qo_len * kv_len) entries, packed into bits on the device
        (bsx_custom_mask_prepare).  Returns (mask mode, descriptor, tree words):
        BSX_MASK_TREE with one word per query token when every request's mask sees its
        prefix and has at most 32 query tokens; else BSX_MASK_CUSTOM with the packed bits.
        One host read of the per-request verdicts (a few bytes), no copy of the mask."""
        dev = self._device
        batch = int(qo_lens.shape[0])
        need = int(np.sum(qo_lens.astype(np.int64) * kv_lens.astype(np.int64)))
        m = custom_mask.reshape(-1)
        if m.numel() < need:
            raise ValueError(f"custom_mask has {m.numel()} entries, the page table needs {need}")
        if need >= 2 ** 31:
            raise NotImplementedError("custom masks of 2^31 entries or more")
        if m.device != dev:
            m = m.to(dev)
        if m.dtype != torch.bool:
            m = m != 0
        m = m.contiguous()
        off = np.zeros(batch, np.int64)
        if batch > 1:
            off[1:] = np.cumsum(qo_lens.astype(np.int64) * kv_lens.astype(np.int64))[:-1]
        req = np.stack([qo_h[:-1].astype(np.int64), qo_lens, kv_lens, off], 1).astype(np.int32)
        total_qo = int(qo_h[-1])
        tree = torch.empty(max(total_qo, 1), dtype=torch.int32, device=dev)
        desc = torch.empty(batch + (need + 31) // 32 + 1, dtype=torch.int32, device=dev)
        general = torch.empty(max(batch, 1), dtype=torch.int32, device=dev)
        with torch.cuda.device(dev):
            req_d = torch.from_numpy(req).to(dev)
            rc = _lib.load().bsx_custom_mask_prepare(m.data_ptr(), need, req_d.data_ptr(), batch,
                                                     desc.data_ptr(), tree.data_ptr(),
                                                     general.data_ptr(), stream_of(dev))
            _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.plan(custom_mask)")
            verdict = general[:batch].cpu().numpy()
        if np.any(verdict == 2):
            raise ValueError("custom_mask entries of a request lie outside the mask")
        if np.any(verdict == 1):
            if self._use_cuda_graph:
                raise NotImplementedError(
                    "graph-mode plans take custom masks whose rows see every prefix token "
                    "and that have at most 32 query tokens per request")
            return _lib.MASK_CUSTOM, desc, None
        return _lib.MASK_TREE, None, tree[:total_qo]

    def _host_tables(self, *tables: torch.Tensor) -> list:
        """Host int32 copies of the page-table arrays the host planner reads.  Device
        tensors are copied on the current stream into one pinned staging buffer and read
        after a single synchronisation (a copy per array would synchronise per array)."""
        if not all(t.is_cuda for t in tables):
            return [_host_i32(t) for t in tables]
        sizes = [t.numel() for t in tables]
        total = sum(sizes)
        if self._pinned_tab is None or self._pinned_tab.numel() < total:
            self._pinned_tab = torch.empty(max(total, 4096), dtype=torch.int32, pin_memory=True)
        with torch.cuda.device(tables[0].device):
            off = 0
            for t, n in zip(tables, sizes):
                src = t.detach().reshape(-1)
                if src.dtype != torch.int32:
                    src = src.to(torch.int32)
                self._pinned_tab[off:off + n].copy_(src, non_blocking=True)
                off += n
            torch.cuda.current_stream().synchronize()
        out, off = [], 0
        for n in sizes:
            out.append(self._pinned_tab[off:off + n].numpy().copy())
            off += n
        return out

    def _fixed_shape(self, lib, batch: int, max_qo: int, static: tuple) -> _lib.AttnPlan:
        """The bound-sized shape of graph mode: kept while plans fit it (same heads, page
        size and mask; at most its requests and query tokens per request).  Returns the
        shape without adopting it: plan() adopts it once the plan is accepted."""
        shp = self._graph_shape
        if shp is not None and self._graph_static == static and batch <= shp.batch \
                and max(max_qo, 1) <= shp.max_qo_len:
            return shp
        cap_b = batch
        if self._qo_indptr_buf is not None:
            cap_b = max(cap_b, self._qo_indptr_buf.numel() - 1)
        if shp is not None and self._graph_static == static:
            cap_b = max(cap_b, int(shp.batch))
            max_qo = max(max_qo, int(shp.max_qo_len))
        nq, nk, d, ps, mode, sink, window, scale = static
        new = _lib.AttnPlan()
        rc = lib.bsx_attn_plan_device_shape(max(cap_b, 1), nq, nk, d, ps, mode, sink, window, scale,
                                            self._num_cus, max(max_qo, 1), ctypes.byref(new))
        _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.plan")
        return new

    @staticmethod
    def _launch_sig(plan: _lib.AttnPlan, blob_bytes: int) -> tuple:
        return tuple(getattr(plan, n) for n, _ in plan._fields_
                     if n not in ("total_qo", "total_tiles")) + (blob_bytes,)

    def _check_captured(self, plan: _lib.AttnPlan, blob_bytes: int) -> None:
        """In graph mode a captured run() replays with the launch arguments and the q /
        out / lse buffers it was captured with; a plan that would need other arguments,
        or more query token rows than those buffers hold, is refused instead of being
        replayed stale (or past the buffers' ends)."""
        if self._captured_sig is None:
            return
        if self._launch_sig(plan, blob_bytes) != self._captured_sig:
            raise ValueError(
                "plan(): a graph captured run() of this wrapper, and this plan needs a larger "
                "fixed shape (more requests or query tokens per request, or other heads / mask); "
                "pass max_qo_len= to the first plan() or use a new wrapper for the new shape")
        if int(plan.total_qo) > self._captured_rows:
            raise ValueError(
                f"plan(): a graph captured run() with q / out of {self._captured_rows} token "
                f"rows, and this plan has {int(plan.total_qo)} query tokens; capture run() with "
                "buffers sized for the largest step")

    @property
    def plan_blob(self) -> Optional[np.ndarray]:
        """Host copy of the last host plan's schedule blob (None after a device plan)."""
        return self._host_blob

    def _set_kv_indices(self, paged_kv_indices: torch.Tensor, non_blocking: bool) -> None:
        # Page ids: in graph mode run() reads the registered buffer.
        if self._use_cuda_graph:
            nidx = paged_kv_indices.numel()
            if nidx > self._kv_indices_buf.numel():
                raise ValueError("paged_kv_indices larger than paged_kv_indices_buf")
            if paged_kv_indices.data_ptr() != self._kv_indices_buf.data_ptr():
                self._kv_indices_buf[:nidx].copy_(paged_kv_indices, non_blocking=non_blocking)
            self._kv_indices = self._kv_indices_buf
        else:
            self._kv_indices = paged_kv_indices
        require_gpu("plan", self._kv_indices)
        if self._kv_indices.dtype != torch.int32:
            raise ValueError("paged_kv_indices must be int32")

    def _set_mask_words(self, words, rows: int) -> None:
        if isinstance(words, torch.Tensor):
            w = words.view(torch.int32) if words.dtype in (torch.int32, torch.uint32) \
                else words.to(torch.int32)
        else:
            w = torch.from_numpy(np.ascontiguousarray(
                np.asarray(words, dtype=np.uint32).view(np.int32)))
        if w.numel() < rows:
            raise ValueError("tree_mask_words needs one word per query token")
        w = w.reshape(-1)[:rows]
        self._mask_buffer(w.numel())[: w.numel()].copy_(w, non_blocking=True)

    def _mask_buffer(self, rows: int) -> torch.Tensor:
        """The per-token mask-word buffer, at least `rows` words (fixed in graph mode)."""
        if self._mask_words is None or self._mask_words.numel() < rows:
            if self._use_cuda_graph and self._mask_words is not None:
                raise ValueError("mask grew beyond its cuda-graph buffer")
            cap = max(rows, 1)
            if self._use_cuda_graph and self._qo_indptr_buf is not None:
                cap = max(cap, 32 * (self._qo_indptr_buf.numel()))
            cmb = self._custom_mask_buf
            if self._use_cuda_graph and cmb is not None and cmb.is_cuda \
                    and cmb.device == self._device and cmb.is_contiguous() \
                    and cmb.data_ptr() % 4 == 0 and cmb.numel() * cmb.element_size() >= 4 * cap:
                # graph mode: the per-token words live in the caller's fixed mask buffer
                # (FlashInfer packs its bit mask there), one int32 per query token
                self._mask_words = cmb.view(torch.uint8).reshape(-1)[: 4 * cap].view(torch.int32)
            else:
                self._mask_words = torch.zeros(cap, dtype=torch.int32, device=self._device)
        return self._mask_words

    def _plan_on_device(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len,
                        num_qo_heads, num_kv_heads, head_dim, page_size, custom_mask, causal,
                        sm_scale, qdt, tree_mask_words, sink_tokens, window_tokens, max_qo_len,
                        non_blocking) -> None:
        if max_qo_len is None or int(max_qo_len) < 1:
            raise ValueError("plan(on_device=True) needs max_qo_len >= 1")
        if custom_mask is not None:
            raise NotImplementedError("plan(on_device=True) takes tree_mask_words, not custom_mask")
        streaming = sink_tokens > 0 or window_tokens > 0
        if tree_mask_words is not None:
            if causal or streaming:
                raise ValueError("tree mask cannot be combined with causal or streaming")
            mode = _lib.MASK_TREE
        elif streaming:
            mode = _lib.MASK_STREAMING
        elif causal:
            mode = _lib.MASK_CAUSAL
        else:
            mode = _lib.MASK_NONE
        dev = require_gpu("plan", qo_indptr, paged_kv_indptr, paged_kv_last_page_len)
        batch = qo_indptr.numel() - 1
        if batch < 1 or paged_kv_indptr.numel() != batch + 1 \
                or paged_kv_last_page_len.numel() < batch:
            raise ValueError("qo_indptr, paged_kv_indptr and paged_kv_last_page_len disagree on batch")
        lib = _lib.load()
        plan = _lib.AttnPlan()
        rc = lib.bsx_attn_plan_device_shape(batch, int(num_qo_heads), int(num_kv_heads),
                                            int(head_dim), int(page_size), mode, int(sink_tokens),
                                            int(window_tokens),
                                            float(sm_scale) if sm_scale else 0.0, self._num_cus,
                                            int(max_qo_len), ctypes.byref(plan))
        _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.plan(on_device=True)")
        blob_bytes = _align(int(plan.plan_ints) * 4)
        need = blob_bytes + int(plan.float_ws_bytes)
        if need > self._ws.numel():
            raise ValueError(f"float_workspace_buffer too small: need {need} bytes, "
                             f"have {self._ws.numel()}")
        self._check_captured(plan, blob_bytes)
        self._blob_bytes = blob_bytes
        self._host_blob = None
        self._dev_idx = [t if t.dtype == torch.int32 and t.is_contiguous()
                         else t.to(torch.int32).contiguous()
                         for t in (qo_indptr, paged_kv_indptr, paged_kv_last_page_len)]
        blob = self._ws[: int(plan.plan_ints) * 4]
        rc = lib.bsx_attn_plan_device(ctypes.byref(plan), self._dev_idx[0].data_ptr(),
                                      self._dev_idx[1].data_ptr(), self._dev_idx[2].data_ptr(),
                                      int(paged_kv_indices.numel()), blob.data_ptr(),
                                      stream_of(dev))
        _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.plan(on_device=True)")
        self._set_kv_indices(paged_kv_indices, non_blocking)
        if tree_mask_words is not None:
            self._set_mask_words(tree_mask_words, int(plan.total_qo))
        self._plan = plan
        self._dtype = qdt

    def device_plan_error(self) -> int:
        """Error code the device planner left for the last plan(on_device=True) (0: none;
        reads device memory, so it synchronises)."""
        plan = self._plan
        if plan is None or not plan.device_plan:
            return 0
        return int(self._ws[int(plan.off_dyn) * 4: int(plan.off_dyn) * 4 + 8]
                   .view(torch.int32)[1].item())

    # ------------------------------------------------------------------- run
    def run(self, q: torch.Tensor,
            paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
            out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
            return_lse: bool = False, *, append_key: Optional[torch.Tensor] = None,
            append_value: Optional[torch.Tensor] = None, **unused):
        """Attention output [nnz, num_qo_heads, head_dim] (and lse [nnz, num_qo_heads]).

        With ``append_key`` / ``append_value`` ([nnz, num_kv_heads, head_dim], the cache's
        dtype) the layer's KV update runs in the same call: the rows go to the last qo_len
        positions of each request (StandardKVCache.update with kv_append_indptr =
        qo_indptr, batchspec/models/modules/kv_cache.py:47-84, as
        batchspec/models/modules/attention/standard.py:63-66 calls it) and attention sees
        them, as the update followed by run() does.  The plan's page table must already
        count those tokens (insert_kv runs before the layers).  One launch: the
        attention kernel writes the rows into the cache before reading them."""
        plan = self._plan
        if plan is None:
            raise RuntimeError("plan() must be called before run()")
        k_cache, v_cache, page_stride = _split_cache(paged_kv_cache, plan)
        dev = require_gpu("run", q, k_cache, v_cache)
        if q.dtype != k_cache.dtype or q.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"q ({q.dtype}) and paged_kv_cache ({k_cache.dtype}) must both be "
                             "bf16 or fp16")
        rows_ok = q.shape[0] >= plan.total_qo if plan.device_plan else q.shape[0] == plan.total_qo
        if q.dim() != 3 or tuple(q.shape[1:]) != (plan.num_qo_heads, plan.head_dim) or not rows_ok:
            raise ValueError(f"q shape {tuple(q.shape)} does not match the plan "
                             f"[{plan.total_qo}, {plan.num_qo_heads}, {plan.head_dim}]")
        if q.stride(2) != 1 or q.stride(1) != plan.head_dim:
            q = q.contiguous()
        if out is None:
            out = torch.empty_like(q) if plan.device_plan else torch.empty(
                (plan.total_qo, plan.num_qo_heads, plan.head_dim), dtype=q.dtype, device=dev)
        elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1 \
                or out.stride(1) != plan.head_dim:
            raise ValueError("out must match q in shape and dtype with dense heads")
        if return_lse and lse is None:
            lse = torch.empty((q.shape[0], plan.num_qo_heads), dtype=torch.float32, device=dev)
        if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous()
                                or lse.dim() != 2 or lse.shape[1] != plan.num_qo_heads
                                or lse.shape[0] < plan.total_qo):
            raise ValueError(f"lse must be a contiguous float32 tensor of at least "
                             f"[{plan.total_qo}, {plan.num_qo_heads}]")
        if append_key is not None or append_value is not None:
            kn = _append_rows(append_key, "append_key", q, plan, k_cache.dtype)
            vn = _append_rows(append_value, "append_value", q, plan, k_cache.dtype)
        if q.shape[0] == 0:  # no query token: nothing to attend or to append
            return (out, lse) if return_lse else out
        ws = self._ws
        blob = ws[: int(plan.plan_ints) * 4]
        fws = ws[self._blob_bytes:] if int(plan.float_ws_bytes) > 0 else None
        lib = _lib.load()
        if plan.mask_mode == _lib.MASK_CUSTOM:
            mw = self._custom_desc.data_ptr()
        else:
            mw = (None if self._mask_words is None or plan.mask_mode != _lib.MASK_TREE
                  else self._mask_words.data_ptr())
        if append_key is None and append_value is None:
            rc = lib.bsx_attn_run(ctypes.byref(plan), blob.data_ptr(),
                                  None if fws is None else fws.data_ptr(),
                                  dtype_code(q.dtype), q.data_ptr(), q.stride(0),
                                  k_cache.data_ptr(), v_cache.data_ptr(), page_stride,
                                  self._kv_indices.data_ptr(), mw,
                                  out.data_ptr(), out.stride(0), _lib.ptr(lse), stream_of(dev))
        else:
            rc = lib.bsx_attn_run_append(ctypes.byref(plan), blob.data_ptr(),
                                         None if fws is None else fws.data_ptr(),
                                         dtype_code(q.dtype), q.data_ptr(), q.stride(0),
                                         k_cache.data_ptr(), v_cache.data_ptr(), page_stride,
                                         self._kv_indices.data_ptr(), mw,
                                         out.data_ptr(), out.stride(0), _lib.ptr(lse),
                                         kn.data_ptr(), kn.stride(0), vn.data_ptr(), vn.stride(0),
                                         stream_of(dev))
        _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.run")
        if torch.cuda.is_current_stream_capturing():
            self._captured_sig = self._launch_sig(plan, self._blob_bytes)
            rows = min(q.shape[0], out.shape[0])
            if lse is not None:
                rows = min(rows, lse.shape[0])
            self._captured_rows = rows if self._captured_rows == 0 else min(rows, self._captured_rows)
        return (out, lse) if return_lse else out

    forward = run

    @property
    def plan_info(self) -> Optional[_lib.AttnPlan]:
        return self._plan


def _append_rows(x: Optional[torch.Tensor], name: str, q: torch.Tensor, plan,
                 dtype: torch.dtype) -> torch.Tensor:
    """The appended K or V rows: [q rows, num_kv_heads, head_dim], dense heads, the
    cache's dtype, on q's device."""
    if x is None:
        raise ValueError("append_key and append_value go together")
    shape = (q.shape[0], plan.num_kv_heads, plan.head_dim)
    if tuple(x.shape) != shape or x.dtype != dtype or x.device != q.device:
        raise ValueError(f"{name} must be {list(shape)} {dtype} on {q.device}, got "
                         f"{list(x.shape)} {x.dtype} on {x.device}")
    if x.stride(2) != 1 or x.stride(1) != plan.head_dim or x.stride(0) % 8 != 0 \
            or x.data_ptr() % 16 != 0:
        x = x.contiguous()
    return x


def _as_dtype(d) -> torch.dtype:
    if isinstance(d, torch.dtype):
        return d
    return getattr(torch, str(d).replace("torch.", ""))


def _split_cache(cache, plan) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """(k view, v view, page stride in elements) for the NHD layouts of the reference."""
    H, D, ps = plan.num_kv_heads, plan.head_dim, plan.page_size
    if isinstance(cache, (tuple, list)):
        k, v = cache
        if k.dim() != 4 or tuple(k.shape[1:]) != (ps, H, D) or k.shape != v.shape:
            raise ValueError(f"k/v caches must be [P, {ps}, {H}, {D}]")
        if k.stride()[1:] != (H * D, D, 1) or v.stride() != k.stride():
            raise ValueError("k/v caches must be dense within a page and share strides")
        return k, v, k.stride(0)
    if cache.dim() != 5 or tuple(cache.shape[1:]) != (2, ps, H, D):
        raise ValueError(f"paged_kv_cache must be [P, 2, {ps}, {H}, {D}] (NHD), "
                         f"got {tuple(cache.shape)}")
    if cache.stride()[1:] != (ps * H * D, H * D, D, 1):
        raise ValueError("paged_kv_cache must be dense within a page")
    return cache[:, 0], cache[:, 1], cache.stride(0)
