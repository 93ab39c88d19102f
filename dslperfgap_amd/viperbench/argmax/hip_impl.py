"""ViperBench/argmax - HIP backend.

Unified API of ViperBench/argmax/pytorch_impl.py:4-8:
``argmax(input_tensor, dim, keepdim=False)`` = torch.argmax(input_tensor,
dim=dim, keepdim=keepdim): int64 index of the first maximum (NaN counts as the
largest value); ``dim=None`` flattens (libvbhip ``vbh_reduce_fwd``,
VBH_REDUCE_ARGMAX).
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

from dslperfgap_amd import _lib, _reduce  # noqa: E402


def argmax(input_tensor, dim, keepdim=False):
    """Returns the indices of the maximum values across a specified dimension."""
    x = input_tensor
    if type(dim) is int:  # the common call: a cached plan
        r = _reduce.fast_reduce(x, dim, keepdim, _lib.REDUCE_ARGMAX)
        if r is not None:
            return r[1]
    if dim is None:
        if x.numel() == 0:
            raise IndexError(
                "argmax(): Expected reduction dim to be specified for input.numel() == 0.")
        _, idx = _reduce.reduce(x.reshape(-1), [0], False, _lib.REDUCE_ARGMAX, x.dtype, "argmax")
        return idx.reshape([1] * x.dim()) if keepdim else idx.reshape([])
    dims = _reduce.norm_dims(int(dim), x.dim(), "argmax")
    if x.dim() > 0 and x.shape[dims[0]] == 0:  # other empty axes give an empty result
        raise IndexError(f"argmax(): Expected reduction dim {dims[0]} to have non-zero size.")
    _, idx = _reduce.reduce(x, dims, keepdim, _lib.REDUCE_ARGMAX, x.dtype, "argmax")
    return idx
