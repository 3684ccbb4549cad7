"""The verify path as torch custom operators, so a ``torch.compile``-d forward keeps it.

BatchSpec compiles the engine's forward under its ``--compile`` flag
(batchspec/backends/standard_engine.py:104-106, batchspec/backends/mtp_engine.py:165-169)
and reaches attention and the KV update through registered operators, not Python calls:
the MTP model binds ``torch.ops.mylib.attn_prefill`` / ``attn_draft`` /
``attn_draft_and_verify`` to its layers (batchspec/models/mtp_model.py:82-84) and calls
them as ``op(q, kv_cache)`` (batchspec/models/modules/attention/mtp.py:82-93); the KV
update is ``torch.ops.mylib.update_kv(k, v, kv_append_indptr, kv_cache, kv_page_indices,
kv_page_indptr, kv_page_lastlen, page_size)`` (batchspec/models/README.md:826-860).

A plain Python function that hands ``data_ptr()`` to ctypes makes dynamo break the graph
at every call (or fail under ``fullgraph=True``).  Here each entry point is a
``torch.library.custom_op`` with a fake (meta) implementation, so dynamo and inductor
see an opaque operator with known output shapes:

* ``bind_attention(name, wrapper)`` defines ``torch.ops.bsx.<name>(q, kv_cache)`` (once
  per name) and binds it to a ``BatchPrefillWithPagedKVCacheWrapper``; the op runs that
  wrapper's current plan, so ``plan()`` stays outside the compiled region, as in the
  reference (the engines plan before calling the compiled forward).  Binding another
  wrapper to the same name later re-targets the op without recompiling.  It also defines
  ``torch.ops.bsx.<name>_with_append(q, k, v, kv_cache)``, the layer's update and
  attention in one call (the append fused into the attention launch).
* ``torch.ops.bsx.update_kv(...)``: the fused paged append, mutating ``kv_cache`` in place.
* ``torch.ops.bsx.evaluate_posterior_greedy`` / ``evaluate_posterior_sampling``: the
  acceptance of batchspec/backends/mtp_engine.py:533-575 with its output tuple.
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from .page import append_kv
from .posterior import evaluate_posterior

_WRAPPERS: Dict[str, object] = {}
_DEFINED: Dict[str, object] = {}
_RULES = ("reference", "prefix")


def _attention_op(name: str):
    @torch.library.custom_op(f"bsx::{name}", mutates_args=())
    def op(q: torch.Tensor, kv_cache: torch.Tensor) -> torch.Tensor:
        w = _WRAPPERS.get(name)
        if w is None:
            raise RuntimeError(f"torch.ops.bsx.{name}: no wrapper bound (call bind_attention)")
        return w.run(q, kv_cache)

    @op.register_fake
    def _(q, kv_cache):
        # run() writes one output row per query row: a host plan takes exactly its
        # query tokens, a device or graph-mode plan q's rows (its bound)
        return torch.empty_like(q)

    return op


def _attention_append_op(name: str):
    @torch.library.custom_op(f"bsx::{name}_with_append", mutates_args=("kv_cache",))
    def op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
           kv_cache: torch.Tensor) -> torch.Tensor:
        w = _WRAPPERS.get(name)
        if w is None:
            raise RuntimeError(f"torch.ops.bsx.{name}_with_append: no wrapper bound")
        return w.run(q, kv_cache, append_key=k, append_value=v)

    @op.register_fake
    def _(q, k, v, kv_cache):
        return torch.empty_like(q)

    return op


def bind_attention(name: str, wrapper) -> object:
    """``torch.ops.bsx.<name>(q, kv_cache)`` running ``wrapper.run`` with the wrapper's
    current plan; defines the operator on first use of the name.  Returns the op.  Also
    defines ``torch.ops.bsx.<name>_with_append(q, k, v, kv_cache)``: the layer's KV update
    (k / v at the tail of each request, as update_kv with kv_append_indptr = qo_indptr)
    and its attention in one call, mutating ``kv_cache``."""
    if not name.isidentifier():
        raise ValueError(f"operator name {name!r} must be an identifier")
    if name not in _DEFINED:
        _DEFINED[name] = (_attention_op(name), _attention_append_op(name))
    _WRAPPERS[name] = wrapper
    return getattr(torch.ops.bsx, name)


@torch.library.custom_op("bsx::update_kv", mutates_args=("kv_cache",))
def update_kv(k: torch.Tensor, v: torch.Tensor, kv_append_indptr: torch.Tensor,
              kv_cache: torch.Tensor, kv_page_indices: torch.Tensor,
              kv_page_indptr: torch.Tensor, kv_page_lastlen: torch.Tensor,
              page_size: int) -> None:
    """k / v [nnz, H_kv, D] appended at the tail of each request's pages (positions from
    the page table on the device); ``kv_cache`` [P, 2, page_size, H_kv, D] is updated in
    place."""
    if kv_cache.dim() != 5 or kv_cache.shape[2] != page_size:
        raise ValueError(f"kv_cache must be [P, 2, {page_size}, H, D], got {tuple(kv_cache.shape)}")
    append_kv(k, v, kv_append_indptr, kv_cache, kv_page_indptr, kv_page_indices, kv_page_lastlen)


@update_kv.register_fake
def _(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_page_lastlen,
      page_size):
    return None


@torch.library.custom_op("bsx::evaluate_posterior_greedy", mutates_args=())
def evaluate_posterior_greedy(draft_tokens: torch.Tensor, target_preds: torch.Tensor,
                              eos_token_id: int, accept_rule: int = 0
                              ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Greedy acceptance (mtp_engine.py:553-560): target ids [B, k+1] or logits
    [B, k+1, V] (argmax fused); accept_rule 0 = the reference's count + 1, 1 = longest
    prefix.  Returns (bonus [B, 1] int64, accept_nums [B] int64, eos_accepted [B, 1] bool)."""
    bonus, accept, eos = evaluate_posterior(draft_tokens, target_preds, greedy=True,
                                            eos_token_id=eos_token_id,
                                            accept_rule=_RULES[accept_rule])
    return bonus.clone(), accept, eos.clone()


@evaluate_posterior_greedy.register_fake
def _(draft_tokens, target_preds, eos_token_id, accept_rule=0):
    B = draft_tokens.shape[0]
    dev = draft_tokens.device
    return (torch.empty((B, 1), dtype=torch.int64, device=dev),
            torch.empty((B,), dtype=torch.int64, device=dev),
            torch.empty((B, 1), dtype=torch.bool, device=dev))


@torch.library.custom_op("bsx::evaluate_posterior_sampling", mutates_args=())
def evaluate_posterior_sampling(draft_tokens: torch.Tensor, target_logits: torch.Tensor,
                                eos_token_id: int, temperature: float, top_p: float, top_k: int,
                                uniforms: torch.Tensor
                                ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Sampling acceptance (mtp_engine.py:561-575): filtered target distribution at the
    temperature, one-hot drafts, chain speculative sampling with the caller's uniforms
    [B, k+1].  Returns (bonus [B, 1] int32, accept_nums = emitted + 1 [B] int32,
    eos_accepted [B, 1] bool), the dtypes of the reference's branch."""
    bonus, accept, eos = evaluate_posterior(draft_tokens, target_logits, greedy=False,
                                            eos_token_id=eos_token_id, temperature=temperature,
                                            top_p=top_p, top_k=top_k, uniforms=uniforms)
    return bonus.contiguous(), accept.contiguous(), eos.contiguous()


@evaluate_posterior_sampling.register_fake
def _(draft_tokens, target_logits, eos_token_id, temperature, top_p, top_k, uniforms):
    B = draft_tokens.shape[0]
    dev = draft_tokens.device
    return (torch.empty((B, 1), dtype=torch.int32, device=dev),
            torch.empty((B,), dtype=torch.int32, device=dev),
            torch.empty((B, 1), dtype=torch.bool, device=dev))
