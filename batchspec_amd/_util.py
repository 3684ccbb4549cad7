"""Small helpers shared by the host-side wrappers (device checks, streams, dtypes)."""
from __future__ import annotations

import functools

import torch

from . import _lib

_DTYPE_CODE = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16,
               torch.float32: _lib.DTYPE_FP32}


def dtype_code(dt: torch.dtype, allowed=(torch.bfloat16, torch.float16, torch.float32)) -> int:
    if dt not in allowed:
        raise ValueError(f"unsupported dtype {dt}; expected one of {allowed}")
    return _DTYPE_CODE[dt]


def require_gpu(what: str, *tensors) -> torch.device:
    """All tensors must live on one ROCm GPU: this package has no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError(f"{what}: expected tensors on a ROCm GPU device, got "
                             f"{getattr(t, 'device', type(t))}; batchspec_amd has no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: tensors on different devices ({dev} and {t.device})")
    if dev is None:
        raise ValueError(f"{what}: no tensor given")
    return dev


def stream_of(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (as an integer address)."""
    return torch.cuda.current_stream(device).cuda_stream


@functools.lru_cache(maxsize=None)
def num_cus(device_index: int) -> int:
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def workspace(device: torch.device, nbytes: int, cache: dict | None = None,
              key: str = "ws") -> torch.Tensor:
    """A uint8 device buffer of at least `nbytes`, reused through `cache`.

    A buffer that is outgrown is never freed: a graph captured while it was current
    holds its address as a kernel argument, and replaying that graph must not write
    into memory the caching allocator has handed to another tensor.  Growth doubles,
    so the retired buffers together stay below the current one."""
    nbytes = max(int(nbytes), 256)
    if cache is None:
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    buf = cache.get(key)
    if buf is not None and buf.numel() >= nbytes and buf.device == device:
        return buf
    if buf is not None:
        cache.setdefault("__retired__", []).append(buf)
        nbytes = max(nbytes, 2 * buf.numel())
    buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
    cache[key] = buf
    return buf
