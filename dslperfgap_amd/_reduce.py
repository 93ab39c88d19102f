"""Shared host logic of the axis reductions (mean / max / argmax): dim
normalisation, the [outer, n, inner] view and the output shape.  The compute is
libvbhip's ``vbh_reduce_fwd``."""
from __future__ import annotations

import torch

from . import _bridge, _lib


def norm_dims(dim, ndim: int, what: str) -> list[int]:
    """Sorted, de-duplicated non-negative dims (torch's IndexError / RuntimeError)."""
    n = max(ndim, 1)
    dims = list(range(n)) if dim is None else ([dim] if isinstance(dim, int) else list(dim))
    out = []
    for d in dims:
        d = int(d)
        if not -n <= d < n:
            raise IndexError(f"Dimension out of range (expected to be in range of [{-n}, "
                             f"{n - 1}], but got {d})")
        d %= n
        if d in out:
            raise RuntimeError(f"{what}: dim {d} appears multiple times in the list of dims")
        out.append(d)
    return sorted(out)


def reduce(x: torch.Tensor, dims: list[int], keepdim: bool, op: int, out_dtype, what: str):
    """Run one reduction over `dims` of `x`; returns (values or None, indices or None)."""
    dev = _bridge.require_gpu(what, x)
    idt = _bridge.float_code(x, what)
    odt = _bridge.FLOAT_CODES[out_dtype]
    shape = tuple(x.shape) if x.dim() > 0 else (1,)
    xc = x if x.dim() > 0 else x.reshape(shape)
    if dims[-1] - dims[0] == len(dims) - 1:  # adjacent dims collapse into one axis
        outer = _bridge.numel_prod(shape[:dims[0]])
        n = _bridge.numel_prod(shape[dims[0]:dims[-1] + 1])
        inner = _bridge.numel_prod(shape[dims[-1] + 1:])
        if not xc.is_contiguous():
            xc = xc.contiguous()
    else:
        # reduced dims are not adjacent: move them last (one extra copy pass)
        keep = [d for d in range(len(shape)) if d not in dims]
        xc = xc.permute(keep + dims).contiguous()
        outer = _bridge.numel_prod(shape[d] for d in keep)
        n = _bridge.numel_prod(shape[d] for d in dims)
        inner = 1
    if x.dim() == 0:
        out_shape = []
    elif keepdim:
        out_shape = [1 if d in dims else s for d, s in enumerate(shape)]
    else:
        out_shape = [s for d, s in enumerate(shape) if d not in dims]
    vals = None if op == _lib.REDUCE_ARGMAX else torch.empty(out_shape, dtype=out_dtype,
                                                              device=x.device)
    idx = None if op == _lib.REDUCE_MEAN else torch.empty(out_shape, dtype=torch.int64,
                                                          device=x.device)
    if outer * inner == 0:
        return vals, idx
    with _bridge.device_guard(dev):
        _lib.call("vbh_reduce_fwd", _bridge.ptr(xc), _bridge.ptr(vals), _bridge.ptr(idx), outer,
                  n, inner, idt, odt, op, _bridge.stream(dev))
    return vals, idx
