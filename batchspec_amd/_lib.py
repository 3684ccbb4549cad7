"""ctypes binding of the C ABI in ``include/bsx.h`` (``batchspec_amd/libbsx.so``).

The library is the only compute path of this package: nothing here falls back to
PyTorch or to a CPU implementation.  If the shared library has not been built,
importing the ops raises immediately with the build command to run.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_uint8, c_uint32, c_void_p
from pathlib import Path

LIB_PATH = Path(os.environ.get("BSX_LIB", Path(__file__).resolve().parent / "libbsx.so"))

BSX_OK = 0
BSX_ERR_INVALID = -1
BSX_ERR_CAPACITY = -2
BSX_ERR_UNSUPPORTED = -3
BSX_ERR_HIP = -4

NOALLOC_SCRATCH_BYTES = 4 << 20  # BSX_NOALLOC_SCRATCH_BYTES of include/bsx.h

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2

MASK_NONE = 0
MASK_CAUSAL = 1
MASK_TREE = 2
MASK_STREAMING = 3
MASK_CUSTOM = 4


class AttnPlan(ctypes.Structure):
    """Mirror of ``bsx_attn_plan_t``."""

    _fields_ = [
        ("batch", c_int32),
        ("num_qo_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("page_size", c_int32),
        ("mask_mode", c_int32),
        ("group_size", c_int32),
        ("qrow_tile", c_int32),
        ("qrow_blocks", c_int32),
        ("heads_per_cta", c_int32),
        ("qblocks_per_cta", c_int32),
        ("num_qgroups", c_int32),
        ("num_ctas", c_int32),
        ("num_segments", c_int32),
        ("num_partials", c_int32),
        ("num_split_requests", c_int32),
        ("max_qo_len", c_int32),
        ("tile_tokens", c_int32),
        ("sink_tokens", c_int32),
        ("window_tokens", c_int32),
        ("off_seq", c_int32),
        ("off_seg_indptr", c_int32),
        ("off_segments", c_int32),
        ("off_merge_seqs", c_int32),
        ("off_part_indptr", c_int32),
        ("plan_ints", c_int32),
        ("float_ws_bytes", c_int64),
        ("sm_scale", c_float),
        ("total_qo", c_int32),
        ("safe_page_pos", c_int32),
        ("shared_kv_tiles", c_int32),
        ("total_tiles", c_int64),
        ("device_plan", c_int32),
        ("off_dyn", c_int32),
    ]


_P = c_void_p  # every tensor pointer crosses the ABI as a plain address
_PI32 = POINTER(c_int32)

# name -> (restype, argtypes); must match include/bsx.h exactly.
SIGNATURES = {
    "bsx_last_error": (ctypes.c_char_p, []),
    "bsx_version": (c_int, []),
    "bsx_attn_plan_ints_bound": (c_int64, [c_int, c_int]),
    "bsx_attn_plan": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                              c_float, c_int, c_int64, _P, c_int64, POINTER(AttnPlan)]),
    "bsx_attn_plan_fixed": (c_int, [POINTER(AttnPlan), _P, _P, _P, c_int, c_int64, _P, c_int64,
                                    POINTER(AttnPlan)]),
    "bsx_attn_plan_device_shape": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                           c_float, c_int, c_int, POINTER(AttnPlan)]),
    "bsx_attn_plan_device": (c_int, [POINTER(AttnPlan), _P, _P, _P, c_int64, _P, _P]),
    "bsx_attn_run": (c_int, [POINTER(AttnPlan), _P, _P, c_int, _P, c_int64, _P, _P, c_int64, _P,
                             _P, _P, c_int64, _P, _P]),
    "bsx_attn_run_append": (c_int, [POINTER(AttnPlan), _P, _P, c_int, _P, c_int64, _P, _P, c_int64,
                                    _P, _P, _P, c_int64, _P, _P, c_int64, _P, c_int64, _P]),
    "bsx_get_seq_lens": (c_int, [_P, _P, c_int, c_int, _P, _P]),
    "bsx_get_batch_indices_positions": (c_int, [_P, _P, c_int, c_int, _P, _P, _P]),
    "bsx_append_paged_kv_cache": (c_int, [_P, _P, c_int64, c_int64, _P, _P, c_int, _P, _P, c_int64,
                                          _P, _P, c_int, c_int, c_int, c_int, _P]),
    "bsx_kv_append": (c_int, [_P, _P, c_int64, c_int64, _P, _P, _P, _P, c_int, c_int, _P, _P,
                              c_int64, c_int, c_int, c_int, c_int, _P]),
    "bsx_collate_accepted_kv": (c_int, [_P, _P, c_int, c_int, _P, _P, _P, _P, c_int, c_int64,
                                        c_int, c_int, c_int, c_int, _P]),
    "bsx_argmax_ws_bytes": (c_int64, [c_int64, c_int64]),
    "bsx_argmax": (c_int, [_P, c_int, c_int64, c_int64, c_int64, _P, _P, c_int64, _P]),
    "bsx_accept_greedy_ws_bytes": (c_int64, [c_int, c_int, c_int64]),
    "bsx_accept_greedy": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int64, c_int64, c_int, _P, _P,
                                  _P, _P, c_int64, _P]),
    "bsx_accept_greedy_noalloc": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int64, c_int64, c_int,
                                          _P, _P, _P, _P]),
    "bsx_chain_ws_bytes": (c_int64, [c_int, c_int, c_int64]),
    "bsx_chain_speculative_sampling": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int64, _P, _P, _P,
                                               _P, c_int64, _P]),
    "bsx_chain_speculative_sampling_logits": (c_int, [_P, _P, _P, c_int, c_float, _P, c_int, c_int,
                                                      c_int64, _P, _P, _P, _P, c_int64, _P]),
    "bsx_tree_masks": (c_int, [_P, c_int64, c_int, _P, c_int, _P, _P, _P]),
    "bsx_custom_mask_prepare": (c_int, [_P, c_int64, _P, c_int, _P, _P, _P, _P]),
    "bsx_page_table_update": (c_int, [_P, _P, _P, _P, c_int32, c_int, c_int, c_int, c_int, _P, _P,
                                      _P, _P]),
    "bsx_accept_greedy_delete": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_int64, c_int64, c_int,
                                         _P, _P, _P, _P, c_int64, c_int32, _P, _P, _P, c_int, c_int,
                                         _P, _P, _P]),
    "bsx_filter_ws_bytes": (c_int64, [c_int64]),
    "bsx_chain_filtered_ws_bytes": (c_int64, [c_int, c_int, c_int64]),
    "bsx_chain_speculative_sampling_filtered": (c_int, [_P, _P, _P, c_int, c_float, c_int, c_float,
                                                        _P, c_int, c_int, c_int64, _P, _P, _P, _P,
                                                        c_int64, _P]),
    "bsx_sampling_probs_ws_bytes": (c_int64, [c_int64]),
    "bsx_sampling_probs": (c_int, [_P, c_int, c_float, c_int, c_float, c_int64, c_int64, _P, _P,
                                   c_int64, _P]),
    "bsx_sample_ws_bytes": (c_int64, [c_int64, c_int64]),
    "bsx_sample": (c_int, [_P, c_int, c_float, c_int, c_float, _P, c_int64, c_int64, _P, _P,
                           c_int64, _P]),
    "bsx_read_probe": (c_int, [_P, c_int64, c_int, c_int, _P, _P]),
    "bsx_softmax_ws_bytes": (c_int64, [c_int64]),
    "bsx_softmax": (c_int, [_P, c_int, c_float, c_int64, c_int64, _P, _P, c_int64, _P]),
}

_lib = None


class BsxError(RuntimeError):
    """A bsx entry point returned an error status."""


def load() -> ctypes.CDLL:
    """Load libbsx.so once and bind every entry point; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built: run `python -m batchspec_amd.build` "
            "(the HIP library is the only compute path of batchspec_amd)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise the Python exception matching a bsx status code."""
    if rc == BSX_OK:
        return
    msg = load().bsx_last_error().decode(errors="replace")
    text = f"{what}: {msg}"
    if rc in (BSX_ERR_INVALID, BSX_ERR_CAPACITY):
        raise ValueError(text)
    if rc == BSX_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise BsxError(text)


def ptr(t) -> int | None:
    """Device (or host) address of a tensor, None for None."""
    return None if t is None else t.data_ptr()
