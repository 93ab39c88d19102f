"""Torch-side plumbing shared by the hip_impl modules: dtype codes, device
checks, output allocation, raw pointers and the current HIP stream.  Nothing
here computes.

Every wrapper call pays this host path before its kernel runs, and at the
reference's small shapes (1-4 MB) that path is most of a call's latency, so it
avoids the slow forms of torch's Python API (measured per call):
``torch.empty(shape_tuple, dtype=..., device=...)`` parses for 2.3-4.4 us and
``t.new_empty(shape, dtype=...)`` for 2.1-2.3 us, where ``torch.empty_like``
takes 1.1 us and ``t.new_empty_strided`` 1.2-1.6 us; ``t.device`` builds a
device object per access where ``t.get_device()`` returns an int.
"""
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


def require_gpu(what: str, *tensors: torch.Tensor) -> int:
    """All tensors must live on the same GPU; return its device index."""
    idx = -1
    for t in tensors:
        if t is None:
            continue
        d = t.get_device()
        if d < 0:
            raise ValueError(f"{what}: the HIP backend takes GPU tensors, got one on {t.device}")
        if idx < 0:
            idx = d
        elif d != idx:
            raise ValueError(f"{what}: tensors on different devices (cuda:{idx}, cuda:{d})")
    if idx < 0:
        raise ValueError(f"{what}: no tensor arguments")
    return idx


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def contiguous_strides(shape) -> tuple:
    """Row-major strides (in elements) of `shape`."""
    n = len(shape)
    if n == 1:
        return (1,)
    if n == 2:
        return (max(int(shape[1]), 1), 1)
    st = [1] * n
    for i in range(n - 2, -1, -1):
        st[i] = st[i + 1] * max(int(shape[i + 1]), 1)
    return tuple(st)


def empty(like: torch.Tensor, shape, dtype: torch.dtype | None = None) -> torch.Tensor:
    """A new contiguous tensor of `shape` on `like`'s device, of `dtype` (default:
    `like`'s)."""
    st = contiguous_strides(shape)
    if dtype is None or dtype is like.dtype:
        return like.new_empty_strided(shape, st)
    return like.new_empty_strided(shape, st, dtype=dtype)


# torch's raw current-stream accessor skips building a Stream object per call
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
    lambda idx: torch.cuda.current_stream(idx).cuda_stream)


def stream(dev) -> int:
    """Handle of torch's current stream on `dev` (a torch.device or a device
    index); the library launches there."""
    idx = dev if isinstance(dev, int) else dev.index
    return _raw_stream(torch.cuda.current_device() if idx is None else idx)


# torch's raw current-device accessor (torch.cuda.current_device adds a
# lazy-init check per call; a GPU tensor argument has already initialised it)
_raw_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


class PlanCache(dict):
    """Launch plans of the wrappers' common calls, keyed by what decides them
    (shape, dtype, ...): bounded, and registered with the library's geometry
    caches, so that ``_lib.tune_override`` (which changes launch shapes and
    row splits) clears it."""

    LIMIT = 4096

    def __init__(self):
        super().__init__()
        _lib.GEOMETRY_CACHES.append(self)

    def cache_clear(self):
        self.clear()

    def put(self, key, plan):
        if len(self) >= self.LIMIT:
            self.clear()
        self[key] = plan
        return plan


def launch(name: str, idx: int, *args) -> None:
    """Call entry point `name` with `args` followed by the handle of torch's
    current stream on device `idx` (every launching entry point takes the
    stream last), with that device current during the call; raise
    ``_lib.VbhError`` on a nonzero status."""
    launch_fn(_lib.entry(name), name, idx, *args)


def launch_fn(fn, name: str, idx: int, *args) -> None:
    """:func:`launch` with the bound entry point `fn` (``_lib.entry(name)``)
    already looked up."""
    if idx == _raw_device():
        rc = fn(*args, _raw_stream(idx))
    else:
        with torch.cuda.device(idx):
            rc = fn(*args, _raw_stream(idx))
    if rc != 0:
        raise _lib.VbhError(name, rc, _lib.last_error())


def numel_prod(shape) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


# (shape, dtype) -> (rows, cols, dtype code, entry point) of a last-axis
# softmax / log_softmax on the unsplit row kernel, or False
_SOFTMAX_PLANS = PlanCache()


def softmax_rows_fast(x: torch.Tensor, log_mode: int):
    """Softmax (log_mode 0) or log_softmax (1) over the last axis of a
    contiguous tensor on the current GPU, in its own dtype, through a cached
    plan; None where the call needs the wrapper's general path (other devices
    or layouts, split rows, empty or 0-d tensors, unsupported dtypes, which
    that path also rejects with the proper error)."""
    dt = x.dtype
    p = _SOFTMAX_PLANS.get((x.shape, dt))
    if p is None:
        p = _SOFTMAX_PLANS.put((x.shape, dt), _softmax_plan(x, dt))
    if not p:
        return None
    dev = x.get_device()
    if dev < 0 or dev != _raw_device() or not x.is_contiguous():
        return None
    rows, cols, code, fn = p
    y = torch.empty_like(x)
    rc = fn(x.data_ptr(), y.data_ptr(), rows, cols, code, code, log_mode, _raw_stream(dev))
    if rc != 0:
        raise _lib.VbhError("vbh_softmax_fwd", rc, _lib.last_error())
    return y


def _softmax_plan(x: torch.Tensor, dt):
    code = FLOAT_CODES.get(dt)
    if code is None or x.dim() == 0:
        return False
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    if not rows or _lib.softmax_workspace_bytes(rows, cols, code):
        return False
    return (rows, cols, code, _lib.entry("vbh_softmax_fwd"))
