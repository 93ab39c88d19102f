"""Torch-side plumbing shared by the hip_impl modules: dtype codes, device
checks, raw pointers and the current HIP stream.  Nothing here computes."""
from __future__ import annotations

import torch

from . import _lib

FLOAT_CODES = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}
LABEL_CODES = {torch.int32: _lib.I32, torch.int64: _lib.I64}


def float_code(t: torch.Tensor, what: str) -> int:
    try:
        return FLOAT_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: dtype {t.dtype} is not supported by the HIP backend "
                        "(float32, float16, bfloat16)") from None


def require_gpu(what: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors must live on the same GPU; return that device."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{what}: the HIP backend takes GPU tensors, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{what}: tensors on different devices ({dev}, {t.device})")
    if dev is None:
        raise ValueError(f"{what}: no tensor arguments")
    return dev


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


# torch's raw current-stream accessor skips building a Stream object per call
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(dev: torch.device) -> int:
    """Handle of torch's current stream on `dev` (the library launches there)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


# torch's raw current-device accessor (torch.cuda.current_device adds a
# lazy-init check per call; a GPU tensor argument has already initialised it)
_raw_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def launch(name: str, dev: torch.device, *args) -> None:
    """Call entry point `name` with `args` followed by the handle of torch's
    current stream on `dev` (every launching entry point takes the stream
    last), with `dev` the current device during the call."""
    cur = _raw_device()
    idx = cur if dev.index is None else dev.index
    if idx == cur:
        _lib.call(name, *args, stream(dev) if _raw_stream is None else _raw_stream(cur))
        return
    with torch.cuda.device(idx):
        _lib.call(name, *args, stream(dev))


def numel_prod(shape) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n
