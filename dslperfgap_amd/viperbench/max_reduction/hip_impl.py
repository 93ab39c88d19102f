"""ViperBench/max_reduction - HIP backend.

Unified API of ViperBench/max_reduction/pytorch_impl.py:4-11:
``max_reduction(input, dim, keepdim=False) -> (values, indices)`` =
torch.max(input, dim, keepdim): NaN is the largest value and the first maximal
position is returned (libvbhip ``vbh_reduce_fwd``, VBH_REDUCE_MAX).
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import torch  # noqa: E402

from dslperfgap_amd import _lib, _reduce  # noqa: E402


def max_reduction(input, dim, keepdim=False):
    """Computes max along a specified dimension, returning (values, indices)."""
    if not isinstance(input, torch.Tensor):
        raise TypeError('The input must be a torch.Tensor.')
    if type(dim) is int:  # the common call: a cached plan
        r = _reduce.fast_reduce(input, dim, keepdim, _lib.REDUCE_MAX)
        if r is not None:
            return r
    dims = _reduce.norm_dims(int(dim), input.dim(), "max_reduction")
    if input.dim() > 0 and input.shape[dims[0]] == 0:  # other empty axes: empty result
        raise IndexError(f"max(): Expected reduction dim {dims[0]} to have non-zero size.")
    vals, idx = _reduce.reduce(input, dims, keepdim, _lib.REDUCE_MAX, input.dtype,
                               "max_reduction")
    return (vals, idx)
