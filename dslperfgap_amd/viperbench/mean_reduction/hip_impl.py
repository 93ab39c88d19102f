"""ViperBench/mean_reduction - HIP backend.

Unified API of ViperBench/mean_reduction/pytorch_impl.py:4-8:
``mean_reduction(input_tensor, dim, keepdim=False, dtype=None)`` =
torch.mean(input_tensor, dim, keepdim=keepdim, dtype=dtype): fp32 accumulation,
one read of the input (libvbhip ``vbh_reduce_fwd``, VBH_REDUCE_MEAN).  Adjacent
reduced dims collapse into one axis; non-adjacent ones are moved last first.
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import torch  # noqa: E402

from dslperfgap_amd import _bridge, _lib, _reduce  # noqa: E402


def mean_reduction(input_tensor, dim, keepdim=False, dtype=None):
    """Computes the mean value along specified dimensions."""
    x = input_tensor
    if dtype is None and type(dim) is int:  # the common call: a cached plan
        r = _reduce.fast_reduce(x, dim, keepdim, _lib.REDUCE_MEAN)
        if r is not None:
            return r[0]
    out_dtype = x.dtype if dtype is None else dtype
    if out_dtype not in _bridge.FLOAT_CODES:
        raise TypeError(f"mean_reduction: dtype {out_dtype} is not supported by the HIP backend")
    if out_dtype != x.dtype and not (out_dtype == torch.float32 and
                                     x.dtype in (torch.float16, torch.bfloat16)):
        x = x.to(out_dtype)  # torch.mean casts the input to `dtype` first
    dims = _reduce.norm_dims(dim, x.dim(), "mean_reduction")
    vals, _ = _reduce.reduce(x, dims, keepdim, _lib.REDUCE_MEAN, out_dtype, "mean_reduction")
    return vals
