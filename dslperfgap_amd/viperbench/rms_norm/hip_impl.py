"""ViperBench/rms_norm - HIP backend.

Unified API of ViperBench/rms_norm/pytorch_impl.py:3-10:
``rms_norm(x, normalized_shape, weight, eps=1e-5) -> Tensor``, reducing over
the last ``len(normalized_shape)`` dims:
``((x.float() / sqrt(mean(x.float()**2) + eps)) * weight.float()).to(x.dtype)``.

One read of x and one write of y per call (libvbhip ``vbh_rms_norm_fwd``).
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import torch  # noqa: E402

from dslperfgap_amd import _bridge  # noqa: E402


def rms_norm(x, normalized_shape, weight, eps=1e-5):
    """RMS normalization: y = x / sqrt(mean(x^2) + eps) * weight."""
    dev = _bridge.require_gpu("rms_norm", x, weight)
    k = len(tuple(normalized_shape))
    if k > x.dim():
        raise RuntimeError(f"rms_norm: normalized_shape {tuple(normalized_shape)} has more dims "
                           f"than input {list(x.shape)}")
    dt = _bridge.float_code(x, "rms_norm")
    cols = x.shape[-1] if k == 1 else _bridge.numel_prod(x.shape[x.dim() - k:])
    if weight.numel() != cols:
        raise RuntimeError(f"rms_norm: weight has {weight.numel()} elements, the normalized "
                           f"dims hold {cols}")
    # weight.float() in the golden: any float weight is exact in fp32; keep the
    # x dtype when it matches (no extra pass), else widen the small vector once
    w = weight.contiguous() if weight.dtype in (x.dtype, torch.float32) else weight.float()
    wdt = _bridge.FLOAT_CODES[w.dtype]
    x = x.contiguous()
    y = torch.empty_like(x)
    rows = x.numel() // cols if cols else 0
    _bridge.launch("vbh_rms_norm_fwd", dev, _bridge.ptr(x), _bridge.ptr(w), _bridge.ptr(y), rows,
                   cols, float(eps), dt, wdt)
    return y
