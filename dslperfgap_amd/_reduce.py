"""Shared host logic of the axis reductions (mean / max / argmax): dim
normalisation, the [outer, n, inner] view and the output shape.  The compute is
libvbhip's ``vbh_reduce_fwd``."""
from __future__ import annotations

import functools

import torch

from . import _bridge, _lib


def norm_dims(dim, ndim: int, what: str) -> list[int]:
    """Sorted, de-duplicated non-negative dims (torch's IndexError / RuntimeError)."""
    n = max(ndim, 1)
    if type(dim) is int and -n <= dim < n:  # the common case
        return [dim % n]
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


@functools.lru_cache(maxsize=1024)
def plan(shape: tuple, dims: tuple, keepdim: bool, zero_d: bool, idt: int, op: int) -> tuple:
    """(outer, n, inner, permutation or None, output shape, output strides,
    workspace bytes, entry point) of a reduction over the sorted `dims` of a
    tensor of `shape`.  Adjacent dims collapse into one axis of the contiguous
    [outer, n, inner] view; otherwise the reduced dims are moved last (one
    extra copy pass).  A nonzero workspace size means the launch splits its
    rows (``vbh_reduce_fwd_ws``)."""
    if dims[-1] - dims[0] == len(dims) - 1:
        outer = _bridge.numel_prod(shape[:dims[0]])
        n = _bridge.numel_prod(shape[dims[0]:dims[-1] + 1])
        inner = _bridge.numel_prod(shape[dims[-1] + 1:])
        perm = None
    else:
        keep = tuple(d for d in range(len(shape)) if d not in dims)
        perm = keep + dims
        outer = _bridge.numel_prod(shape[d] for d in keep)
        n = _bridge.numel_prod(shape[d] for d in dims)
        inner = 1
    if zero_d:
        out_shape = ()
    elif keepdim:
        out_shape = tuple(1 if d in dims else s for d, s in enumerate(shape))
    else:
        out_shape = tuple(s for d, s in enumerate(shape) if d not in dims)
    ws = _lib.reduce_workspace_bytes(outer, n, inner, idt, op) if outer * inner else 0
    name = "vbh_reduce_fwd_ws" if ws else "vbh_reduce_fwd"
    return (outer, n, inner, perm, out_shape, _bridge.contiguous_strides(out_shape), ws,
            _lib.entry(name), name)


# an overridden launch geometry changes the split decision
_lib.GEOMETRY_CACHES.append(plan)


def reduce(x: torch.Tensor, dims: list[int], keepdim: bool, op: int, out_dtype, what: str):
    """Run one reduction over `dims` of `x`; returns (values or None, indices or None)."""
    dev = _bridge.require_gpu(what, x)
    idt = _bridge.float_code(x, what)
    odt = _bridge.FLOAT_CODES[out_dtype]
    zero_d = x.dim() == 0
    shape = (1,) if zero_d else tuple(x.shape)
    outer, n, inner, perm, out_shape, out_strides, ws_bytes, fn, name = plan(
        shape, tuple(dims), bool(keepdim), zero_d, idt, op)
    xc = x.reshape(shape) if zero_d else x
    if perm is not None:
        xc = xc.permute(perm)
    if not xc.is_contiguous():
        xc = xc.contiguous()
    if op == _lib.REDUCE_ARGMAX:
        vals = None
    elif out_dtype is x.dtype:
        vals = x.new_empty_strided(out_shape, out_strides)
    else:
        vals = x.new_empty_strided(out_shape, out_strides, dtype=out_dtype)
    idx = None if op == _lib.REDUCE_MEAN else x.new_empty_strided(out_shape, out_strides,
                                                                 dtype=torch.int64)
    if outer * inner == 0:
        return vals, idx
    if ws_bytes:  # few long rows: split each row over several workgroups
        ws = _bridge.empty(x, (ws_bytes,), torch.uint8)
        _bridge.launch_fn(fn, name, dev, xc.data_ptr(), _bridge.ptr(vals), _bridge.ptr(idx),
                          outer, n, inner, idt, odt, op, ws.data_ptr(), ws_bytes)
    else:
        _bridge.launch_fn(fn, name, dev, xc.data_ptr(), _bridge.ptr(vals), _bridge.ptr(idx),
                          outer, n, inner, idt, odt, op)
    return vals, idx


# launch plans of single-dim reductions of contiguous inputs, keyed by
# (shape, dim, keepdim, dtype, op)
_FAST = _bridge.PlanCache()


def fast_reduce(x: torch.Tensor, dim: int, keepdim: bool, op: int):
    """reduce() over one int `dim` of a contiguous tensor on the current GPU
    whose reduced axis is not empty, into outputs of the input's dtype, through
    a cached plan: (values or None, indices or None), or None where the call
    needs the general path (which also raises the errors of invalid calls).
    At the reference's small shapes this host path is most of a call's
    latency, so it makes one pass over the tensor's attributes and calls the
    entry point directly."""
    dt = x.dtype
    p = _FAST.get((x.shape, dim, keepdim, dt, op))
    if p is None:
        p = _fast_plan(x, dim, keepdim, dt, op)
        if p is None:
            return None
    dev = x.get_device()
    if dev < 0 or dev != _raw_device() or not x.is_contiguous():
        return None
    outer, n, inner, out_shape, out_strides, fn, name, idt = p
    if op == REDUCE_MEAN:
        vals = x.new_empty_strided(out_shape, out_strides)
        rc = fn(x.data_ptr(), vals.data_ptr(), None, outer, n, inner, idt, idt, op,
                _raw_stream(dev))
        idx = None
    else:
        vals = None if op == REDUCE_ARGMAX else x.new_empty_strided(out_shape, out_strides)
        idx = x.new_empty_strided(out_shape, out_strides, dtype=torch.int64)
        rc = fn(x.data_ptr(), None if vals is None else vals.data_ptr(), idx.data_ptr(), outer,
                n, inner, idt, idt, op, _raw_stream(dev))
    if rc != 0:
        raise _lib.VbhError(name, rc, _lib.last_error())
    return vals, idx


REDUCE_MEAN, REDUCE_ARGMAX = _lib.REDUCE_MEAN, _lib.REDUCE_ARGMAX
_raw_device, _raw_stream = _bridge._raw_device, _bridge._raw_stream


def _fast_plan(x: torch.Tensor, dim: int, keepdim: bool, dt, op: int):
    """The cached plan of fast_reduce (None: the call takes the general path)."""
    ndim = x.dim()
    idt = _bridge.FLOAT_CODES.get(dt)
    if ndim == 0 or idt is None or not -ndim <= dim < ndim:
        return None
    d = dim % ndim
    shape = tuple(x.shape)
    if shape[d] == 0:
        return None
    outer, n, inner, _perm, out_shape, out_strides, ws, fn, name = plan(
        shape, (d,), bool(keepdim), False, idt, op)
    if ws or outer * inner == 0:
        return None
    return _FAST.put((x.shape, dim, keepdim, dt, op),
                     (outer, n, inner, out_shape, out_strides, fn, name, idt))
