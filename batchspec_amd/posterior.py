"""``evaluate_posterior``: the acceptance call of the verify step.

Same inputs and outputs as MTPEngine.evaluate_posterior
(batchspec/backends/mtp_engine.py:533-575), called at mtp_engine.py:746-749:

* greedy (``target_preds`` = ids [B, k+1], or logits [B, k+1, V] whose argmax is
  fused into the kernel instead of ``target_logits.argmax(-1)``):
  returns (bonus [B,1] int64, accept_nums [B] int64, eos_accepted [B,1] bool) with
  the reference rule accept = (#positions where draft == target)+1
  (mtp_engine.py:556).  ``accept_rule="prefix"`` selects the longest-prefix rule.
* sampling (``target_preds`` = logits [B, k+1, V]): softmax at the temperature with
  the top-p / top-k renormalisation of get_sampling_probs (mtp_engine.py:564),
  one-hot draft probabilities, chain speculative sampling; returns
  (bonus [B,1] int32, accept_nums = emitted+1 [B] int32, eos_accepted [B,1] bool),
  the dtypes of the reference's FlashInfer branch.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from ._util import dtype_code, require_gpu, stream_of, workspace
from .sampling import chain_speculative_sampling_from_logits

_WS: dict = {}
_RULES = {"reference": 0, "prefix": 1}


def evaluate_posterior(draft_tokens: torch.Tensor, target_preds: torch.Tensor, *, greedy: bool,
                       eos_token_id: int, temperature: float = 1.0, top_p: float = 0.0,
                       top_k: int = 0, uniforms: Optional[torch.Tensor] = None,
                       generator: Optional[torch.Generator] = None,
                       accept_rule: str = "reference"
                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, k = draft_tokens.shape
    if greedy:
        return _greedy(draft_tokens, target_preds, eos_token_id, _RULES[accept_rule])
    if target_preds.dim() != 3:
        raise ValueError("sampling acceptance needs target logits [B, k+1, V]")
    out, _, emitted = chain_speculative_sampling_from_logits(
        None, draft_tokens, target_preds, temperature, generator, uniforms=uniforms,
        top_k=top_k, top_p=top_p)
    accept_nums = emitted + 1
    last = (out != -1).to(torch.long) * torch.arange(out.shape[1], device=out.device)
    bonus = out.gather(1, last.argmax(dim=1, keepdim=True))
    eos_accepted = (out == eos_token_id).any(dim=1, keepdim=True)
    return bonus, accept_nums, eos_accepted


def _greedy(draft: torch.Tensor, preds: torch.Tensor, eos: int, mode: int):
    dev = require_gpu("evaluate_posterior", draft, preds)
    B, k = draft.shape
    d = draft.to(torch.int64).contiguous()
    bonus = torch.empty(B, dtype=torch.int64, device=dev)
    accept = torch.empty(B, dtype=torch.int64, device=dev)
    eos_acc = torch.empty(B, dtype=torch.uint8, device=dev)
    lib = _lib.load()
    if preds.dim() == 2:
        if preds.shape != (B, k + 1):
            raise ValueError(f"target ids must be [B, k+1], got {tuple(preds.shape)}")
        ids = preds.to(torch.int64).contiguous()
        rc = lib.bsx_accept_greedy(d.data_ptr(), ids.data_ptr(), None, 0, B, k, 0, int(eos), mode,
                                   bonus.data_ptr(), accept.data_ptr(), eos_acc.data_ptr(), None, 0,
                                   stream_of(dev))
    elif preds.dim() == 3:
        if preds.shape[:2] != (B, k + 1):
            raise ValueError(f"target logits must be [B, k+1, V], got {tuple(preds.shape)}")
        V = preds.shape[2]
        x = preds.contiguous()
        ws = workspace(dev, int(lib.bsx_accept_greedy_ws_bytes(B, k, V)), _WS, f"greedy:{dev}")
        rc = lib.bsx_accept_greedy(d.data_ptr(), None, x.data_ptr(), dtype_code(x.dtype), B, k, V,
                                   int(eos), mode, bonus.data_ptr(), accept.data_ptr(),
                                   eos_acc.data_ptr(), ws.data_ptr(), ws.numel(), stream_of(dev))
    else:
        raise ValueError("target_preds must be ids [B, k+1] or logits [B, k+1, V]")
    _lib.check(rc, "evaluate_posterior")
    # the kernel writes 0/1 bytes: a bool view, no conversion kernel
    return bonus[:, None], accept, eos_acc.view(torch.bool)[:, None]


def evaluate_posterior_and_delete(draft_tokens: torch.Tensor, target_preds: torch.Tensor,
                                  page_table, n_inserted: int, *, eos_token_id: int,
                                  accept_rule: str = "reference"
                                  ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Greedy ``evaluate_posterior`` (mtp_engine.py:553-560) followed by
    ``page_table.delete_kv(n_inserted - accept_nums)`` (page_table.py:95-137), the
    verify step's next operation, in one argmax launch (for logits) and one kernel that
    evaluates every request and updates the DevicePageTable.  Same outputs and table
    state as the two calls in sequence; n_inserted >= k + 1 is the number of tokens the
    step inserted per request."""
    dev = require_gpu("evaluate_posterior_and_delete", draft_tokens, target_preds)
    B, k = draft_tokens.shape
    if page_table.max_batch_size != B:
        raise ValueError(f"page table holds {page_table.max_batch_size} requests, drafts {B}")
    d = draft_tokens.to(torch.int64).contiguous()
    bonus = torch.empty(B, dtype=torch.int64, device=dev)
    accept = torch.empty(B, dtype=torch.int64, device=dev)
    eos_acc = torch.empty(B, dtype=torch.uint8, device=dev)
    lib = _lib.load()
    ids = logits = None
    V, dt, ws = 0, 0, None
    if target_preds.dim() == 2:
        if target_preds.shape != (B, k + 1):
            raise ValueError(f"target ids must be [B, k+1], got {tuple(target_preds.shape)}")
        ids = target_preds.to(torch.int64).contiguous()
    elif target_preds.dim() == 3:
        if target_preds.shape[:2] != (B, k + 1):
            raise ValueError(f"target logits must be [B, k+1, V], got {tuple(target_preds.shape)}")
        logits = target_preds.contiguous()
        V, dt = logits.shape[2], dtype_code(logits.dtype)
        ws = workspace(dev, int(lib.bsx_accept_greedy_ws_bytes(B, k, V)), _WS, f"greedy:{dev}")
    else:
        raise ValueError("target_preds must be ids [B, k+1] or logits [B, k+1, V]")
    pt = page_table
    rc = lib.bsx_accept_greedy_delete(
        d.data_ptr(), _lib.ptr(ids), _lib.ptr(logits), dt, B, k, V, int(eos_token_id),
        _RULES[accept_rule], bonus.data_ptr(), accept.data_ptr(), eos_acc.data_ptr(),
        _lib.ptr(ws), 0 if ws is None else ws.numel(), int(n_inserted),
        pt.page_manager.num_allocated_pages.data_ptr(), pt.paged_kv_last_page_len.data_ptr(),
        pt.cachelens.data_ptr(), pt.page_size, pt.max_num_pages_per_request,
        pt.paged_kv_indptr.data_ptr(), pt.paged_kv_indices.data_ptr(), stream_of(dev))
    _lib.check(rc, "evaluate_posterior_and_delete")
    return bonus[:, None], accept, eos_acc.view(torch.bool)[:, None]


class PosteriorMixin:
    """Engine mixin with the reference's method signature; reads ``greedy``,
    ``eos_token_id``, ``temperature``, ``top_p``, ``top_k`` from the engine."""

    accept_rule = "reference"

    def evaluate_posterior(self, draft_tokens: torch.Tensor, target_preds: torch.Tensor):
        return evaluate_posterior(draft_tokens, target_preds, greedy=self.greedy,
                                  eos_token_id=self.eos_token_id,
                                  temperature=getattr(self, "temperature", 1.0),
                                  top_p=getattr(self, "top_p", 0.0),
                                  top_k=getattr(self, "top_k", 0),
                                  uniforms=getattr(self, "posterior_uniforms", None),
                                  accept_rule=self.accept_rule)
