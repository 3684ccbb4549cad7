"""Acceptance and sampling surfaces of the verify step.

* ``chain_speculative_sampling`` — the FlashInfer call at
  batchspec/backends/mtp_engine.py:569 (same positional arguments and 3-tuple
  result), plus an explicit ``uniforms`` tensor [B, k+1]: ``uniforms[:, i]`` drives
  the ratio test of draft position i and ``uniforms[:, k]`` the single residual /
  bonus draw.  Given the same uniforms the token ids are bit-identical to the CPU
  restatement of the algorithm.
* ``chain_speculative_sampling_from_logits`` — the same test fused with the
  temperature softmax of both distributions (reads bf16 logits once).
* ``softmax`` — flashinfer.sampling.softmax as used at
  batchspec/backends/utils/sampling.py:48.
* ``argmax`` — batchspec/backends/utils/sampling.py:89-90 (greedy ``sample``).
* ``get_sampling_probs`` — batchspec/backends/utils/sampling.py:18-58: softmax at the
  temperature, then top-p renormalisation (top_p > 0), then top-k (top_k > 0).
* ``sample`` — batchspec/backends/utils/sampling.py:61-115 with an explicit uniform
  per row (greedy at temperature 0).
Top-k / top-p keep every value at or above a threshold (ties kept): top-p on the full
distribution, then top-k on the renormalised one (the reference's order); top-p >= 1
and top-k >= vocab keep everything.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from ._util import dtype_code, require_gpu, stream_of, workspace

_WS: dict = {}


def _ws(dev: torch.device, nbytes: int, key: str) -> torch.Tensor:
    return workspace(dev, nbytes, _WS, f"{key}:{dev}")


def _uniforms(B: int, k: int, dev, uniforms: Optional[torch.Tensor],
              generator: Optional[torch.Generator]) -> torch.Tensor:
    if uniforms is None:
        return torch.rand((B, k + 1), dtype=torch.float32, device=dev, generator=generator)
    if uniforms.shape != (B, k + 1) or uniforms.dtype != torch.float32:
        raise ValueError(f"uniforms must be float32 [{B}, {k + 1}], got {uniforms.dtype} "
                         f"{tuple(uniforms.shape)}")
    return uniforms.contiguous()


def _accumulate(out: Optional[torch.Tensor], val: torch.Tensor) -> torch.Tensor:
    # FlashInfer adds into caller-provided counters (statistics across steps)
    if out is None:
        return val
    out += val.to(out.dtype)
    return out


def chain_speculative_sampling(draft_probs: Optional[torch.Tensor], draft_token_ids: torch.Tensor,
                               target_probs: torch.Tensor,
                               maybe_output_accepted_token_num: Optional[torch.Tensor] = None,
                               maybe_output_emitted_draft_token_num: Optional[torch.Tensor] = None,
                               deterministic: bool = True,
                               generator: Optional[torch.Generator] = None, *,
                               uniforms: Optional[torch.Tensor] = None
                               ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Chain rejection sampling over fp32 probabilities.

    draft_probs [B, k, V] (None = one-hot at the draft tokens), draft_token_ids
    [B, k], target_probs [B, k+1, V].  Returns output_token_ids [B, k+1] int32
    (-1 after the emitted token), accepted_num [B] int32 (positions that pass the
    test on their own), emitted_num [B] int32 (accepted prefix length)."""
    dev = require_gpu("chain_speculative_sampling", draft_token_ids, target_probs, draft_probs)
    B, k = draft_token_ids.shape
    if target_probs.dim() != 3 or target_probs.shape[:2] != (B, k + 1):
        raise ValueError(f"target_probs must be [B, k+1, V], got {tuple(target_probs.shape)}")
    V = target_probs.shape[2]
    if target_probs.dtype != torch.float32:
        raise ValueError("target_probs must be float32")
    if draft_probs is not None and (draft_probs.shape != (B, k, V) or draft_probs.dtype != torch.float32):
        raise ValueError("draft_probs must be float32 [B, k, V]")
    ids = draft_token_ids.to(torch.int64).contiguous()
    u = _uniforms(B, k, dev, uniforms, generator)
    out = torch.empty((B, k + 1), dtype=torch.int32, device=dev)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    emi = torch.empty(B, dtype=torch.int32, device=dev)
    lib = _lib.load()
    need = int(lib.bsx_chain_ws_bytes(B, k, V))
    ws = _ws(dev, need, "chain")
    tp = target_probs.contiguous()
    dp = None if draft_probs is None else draft_probs.contiguous()
    rc = lib.bsx_chain_speculative_sampling(_lib.ptr(dp), ids.data_ptr(), tp.data_ptr(),
                                            u.data_ptr(), B, k, V, out.data_ptr(), acc.data_ptr(),
                                            emi.data_ptr(), ws.data_ptr(), ws.numel(),
                                            stream_of(dev))
    _lib.check(rc, "chain_speculative_sampling")
    return (out, _accumulate(maybe_output_accepted_token_num, acc),
            _accumulate(maybe_output_emitted_draft_token_num, emi))


def chain_speculative_sampling_from_logits(draft_logits: Optional[torch.Tensor],
                                           draft_token_ids: torch.Tensor,
                                           target_logits: torch.Tensor, temperature: float = 1.0,
                                           generator: Optional[torch.Generator] = None, *,
                                           uniforms: Optional[torch.Tensor] = None,
                                           top_k: int = 0, top_p: float = 1.0
                                           ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``chain_speculative_sampling(get_sampling_probs(draft), ids,
    get_sampling_probs(target))`` over bf16/fp16/fp32 logits without materialising
    probabilities; draft_logits None means one-hot draft probabilities (the MTP case,
    batchspec/backends/mtp_engine.py:565-567).  top_k / top_p filter both
    distributions (sampling.py:50-56)."""
    dev = require_gpu("chain_speculative_sampling_from_logits", draft_token_ids, target_logits,
                      draft_logits)
    B, k = draft_token_ids.shape
    if target_logits.dim() != 3 or target_logits.shape[:2] != (B, k + 1):
        raise ValueError(f"target_logits must be [B, k+1, V], got {tuple(target_logits.shape)}")
    V = target_logits.shape[2]
    if draft_logits is not None and (draft_logits.shape != (B, k, V)
                                     or draft_logits.dtype != target_logits.dtype):
        raise ValueError("draft_logits must be [B, k, V] with the target dtype")
    if not temperature > 0:
        raise ValueError("temperature must be > 0 (greedy acceptance: evaluate_posterior)")
    ids = draft_token_ids.to(torch.int64).contiguous()
    u = _uniforms(B, k, dev, uniforms, generator)
    out = torch.empty((B, k + 1), dtype=torch.int32, device=dev)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    emi = torch.empty(B, dtype=torch.int32, device=dev)
    lib = _lib.load()
    ws = _ws(dev, int(lib.bsx_chain_filtered_ws_bytes(B, k, V)), "chain")
    tl = target_logits.contiguous()
    dl = None if draft_logits is None else draft_logits.contiguous()
    rc = lib.bsx_chain_speculative_sampling_filtered(
        _lib.ptr(dl), ids.data_ptr(), tl.data_ptr(), dtype_code(tl.dtype), float(temperature),
        int(top_k), float(top_p), u.data_ptr(), B, k, V, out.data_ptr(), acc.data_ptr(),
        emi.data_ptr(), ws.data_ptr(), ws.numel(), stream_of(dev))
    _lib.check(rc, "chain_speculative_sampling_from_logits")
    return out, acc, emi


def softmax(logits: torch.Tensor, temperature: Optional[float] = None,
            enable_pdl: Optional[bool] = None) -> torch.Tensor:
    """softmax(logits / temperature) over the last dim, fp32, deterministic order."""
    dev = require_gpu("softmax", logits)
    V = logits.shape[-1]
    x = logits.contiguous()
    rows = x.numel() // V
    T = 1.0 if temperature is None else float(temperature)
    if not T > 0:
        raise ValueError("temperature must be > 0")
    probs = torch.empty(logits.shape, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = _ws(dev, int(lib.bsx_softmax_ws_bytes(rows)), "softmax")
    rc = lib.bsx_softmax(x.data_ptr(), dtype_code(x.dtype), T, rows, V, probs.data_ptr(),
                         ws.data_ptr(), ws.numel(), stream_of(dev))
    _lib.check(rc, "softmax")
    return probs


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """torch.argmax(logits, dim=-1) (first maximum; NaN counts as maximum), int64."""
    dev = require_gpu("argmax", logits)
    V = logits.shape[-1]
    x = logits.contiguous()
    rows = x.numel() // V
    out = torch.empty(logits.shape[:-1], dtype=torch.int64, device=dev)
    lib = _lib.load()
    ws = _ws(dev, int(lib.bsx_argmax_ws_bytes(rows, V)), "argmax")
    rc = lib.bsx_argmax(x.data_ptr(), dtype_code(x.dtype), rows, V, V, out.data_ptr(),
                        ws.data_ptr(), ws.numel(), stream_of(dev))
    _lib.check(rc, "argmax")
    return out


def _flatten(logits: torch.Tensor) -> Tuple[torch.Tensor, int, int]:
    if logits.dim() == 2:
        return logits, logits.shape[0], 1
    if logits.dim() == 3:
        B, S, V = logits.shape
        return logits.reshape(-1, V), B, S
    raise ValueError(f"Given `logits` has an invalid shape: {logits.shape}")


def get_sampling_probs(logits: torch.Tensor, top_p: float, top_k: int,
                       temperature: float) -> torch.Tensor:
    """Probabilities [B, S, V] (fp32) of softmax(logits / T) after the top-p and top-k
    renormalisation of sampling.py:50-56."""
    flat, B, S = _flatten(logits)
    dev = require_gpu("get_sampling_probs", flat)
    if not temperature > 0:
        raise ValueError("temperature must be > 0")
    x = flat.contiguous()
    rows, V = x.shape
    probs = torch.empty((rows, V), dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = _ws(dev, int(lib.bsx_sampling_probs_ws_bytes(rows)), "probs")
    rc = lib.bsx_sampling_probs(x.data_ptr(), dtype_code(x.dtype), float(temperature), int(top_k),
                                float(top_p), rows, V, probs.data_ptr(), ws.data_ptr(), ws.numel(),
                                stream_of(dev))
    _lib.check(rc, "get_sampling_probs")
    return probs.reshape(B, S, V)


def sample(logits: torch.Tensor, top_p: float, top_k: int, temperature: float, *,
           uniforms: Optional[torch.Tensor] = None,
           generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """Token ids [B, S] int64 (sampling.py:61-115): argmax at temperature 0, else one draw
    per row from the filtered distribution driven by ``uniforms`` [B*S] (or [B, S])
    fp32 in [0, 1) (drawn from ``generator`` when not given)."""
    flat, B, S = _flatten(logits)
    if temperature == 0:
        return argmax(flat).reshape(B, S)
    dev = require_gpu("sample", flat)
    if not temperature > 0:
        raise ValueError("temperature must be >= 0")
    x = flat.contiguous()
    rows, V = x.shape
    if uniforms is None:
        u = torch.rand(rows, dtype=torch.float32, device=dev, generator=generator)
    else:
        if uniforms.numel() != rows or uniforms.dtype != torch.float32:
            raise ValueError(f"uniforms must be float32 with {rows} elements")
        u = uniforms.reshape(rows).contiguous()
    ids = torch.empty(rows, dtype=torch.int32, device=dev)
    lib = _lib.load()
    ws = _ws(dev, int(lib.bsx_sample_ws_bytes(rows, V)), "sample")
    rc = lib.bsx_sample(x.data_ptr(), dtype_code(x.dtype), float(temperature), int(top_k),
                        float(top_p), u.data_ptr(), rows, V, ids.data_ptr(), ws.data_ptr(),
                        ws.numel(), stream_of(dev))
    _lib.check(rc, "sample")
    return ids.reshape(B, S).long()
