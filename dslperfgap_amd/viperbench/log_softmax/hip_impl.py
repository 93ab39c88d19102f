"""ViperBench/log_softmax - HIP backend.

Unified API of ViperBench/log_softmax/pytorch_impl.py:4-8:
``log_softmax(x, dim=-1, dtype=None) -> Tensor`` = F.log_softmax(x, dim, dtype).

``dtype`` casts the input before the computation, as F.log_softmax does.  A
widening cast (fp16/bf16 -> fp32) is exact, so the kernel reads the narrow
input directly and writes fp32; any other cast is applied to x first.
The last dim uses the row kernel (``vbh_softmax_fwd``, log_mode 1; few long
rows split through ``vbh_softmax_fwd_ws``); other dims
use the middle-axis kernel (``vbh_softmax_dim_fwd``) on the [outer, n, inner]
view, as the reference's Triton kernel does with its (M, N, K) strides
(ViperBench/log_softmax/triton_impl.py:72-90).
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import torch  # noqa: E402

from dslperfgap_amd import _bridge, _lib  # noqa: E402


def log_softmax(x, dim=-1, dtype=None):
    """Log-softmax: y = log(softmax(x, dim))."""
    if dtype is None and dim == -1:  # the common call, straight to the row kernel
        y = _bridge.softmax_rows_fast(x, 1)
        if y is not None:
            return y
    dev = _bridge.require_gpu("log_softmax", x)
    out_dtype = x.dtype if dtype is None else dtype
    if out_dtype != x.dtype:
        widening = out_dtype == torch.float32 and x.dtype in (torch.float16, torch.bfloat16)
        if not widening:
            x = x.to(out_dtype)
    idt = _bridge.float_code(x, "log_softmax")
    if out_dtype not in _bridge.FLOAT_CODES:
        raise TypeError(f"log_softmax: dtype {out_dtype} is not supported by the HIP backend")
    odt = _bridge.FLOAT_CODES[out_dtype]
    ndim = max(x.dim(), 1)
    if not -ndim <= dim < ndim:
        raise IndexError(f"Dimension out of range (expected to be in range of [{-ndim}, "
                         f"{ndim - 1}], but got {dim})")
    d = dim % ndim
    x = x.contiguous()
    y = torch.empty_like(x) if out_dtype == x.dtype else torch.empty_like(x, dtype=out_dtype)
    shape = list(x.shape) if x.dim() > 0 else [1]
    if d == ndim - 1:
        cols = shape[-1]
        rows = x.numel() // cols if cols else 0
        ws_bytes = _lib.softmax_workspace_bytes(rows, cols, idt) if rows else 0
        if ws_bytes:  # few long rows: split each row over several workgroups
            ws = _bridge.empty(x, (ws_bytes,), torch.uint8)
            _bridge.launch("vbh_softmax_fwd_ws", dev, x.data_ptr(), y.data_ptr(), rows, cols,
                           idt, odt, 1, ws.data_ptr(), ws_bytes)
        else:
            _bridge.launch("vbh_softmax_fwd", dev, _bridge.ptr(x), _bridge.ptr(y), rows, cols,
                           idt, odt, 1)
    else:
        outer = _bridge.numel_prod(shape[:d])
        inner = _bridge.numel_prod(shape[d + 1:])
        _bridge.launch("vbh_softmax_dim_fwd", dev, _bridge.ptr(x), _bridge.ptr(y), outer,
                       shape[d], inner, idt, odt, 1)
    return y
