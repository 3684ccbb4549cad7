"""batchspec_amd — MI355X (gfx950) speculative-verification hot path for BatchSpec.

Drop-in names for the FlashInfer entry points BatchSpec calls on its verify path:

* ``BatchPrefillWithPagedKVCacheWrapper``  (plan/run; paged-KV verify attention)
* ``get_seq_lens``, ``get_batch_indices_positions``, ``append_paged_kv_cache``
  (paged KV append) and ``StandardKVCache``
* ``sampling.chain_speculative_sampling``, ``sampling.softmax`` and the fused
  ``evaluate_posterior`` (acceptance)
* ``ops``: the same entry points as torch custom operators (``torch.ops.bsx.*``), so a
  ``torch.compile``-d forward keeps them in one graph

All compute runs in ``libbsx.so`` (hand-written HIP for gfx950, C ABI in
``include/bsx.h``); the Python layer only validates, plans and launches.
"""
from .attention import BatchPrefillWithPagedKVCacheWrapper
from .page import (StandardKVCache, append_kv, append_paged_kv_cache,
                   get_batch_indices_positions, get_seq_lens)
from .page_table import DevicePageTable
from .posterior import PosteriorMixin, evaluate_posterior, evaluate_posterior_and_delete
from . import masks, ops, sampling

__all__ = [
    "BatchPrefillWithPagedKVCacheWrapper",
    "StandardKVCache",
    "append_kv",
    "append_paged_kv_cache",
    "get_batch_indices_positions",
    "get_seq_lens",
    "DevicePageTable",
    "PosteriorMixin",
    "evaluate_posterior",
    "evaluate_posterior_and_delete",
    "masks",
    "ops",
    "sampling",
]
