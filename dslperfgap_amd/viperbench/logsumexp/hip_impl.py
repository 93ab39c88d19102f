"""ViperBench/logsumexp - HIP backend.

Unified API of ViperBench/logsumexp/pytorch_impl.py:3-5:
``logsumexp(x) -> Tensor`` = torch.logsumexp(x, dim=-1): shape ``x.shape[:-1]``
(0-d for a 1-D input), same dtype as x.

One read of x per call (libvbhip ``vbh_logsumexp_fwd``).  A launch of few
long rows goes through ``vbh_logsumexp_fwd_ws`` with a small workspace: each
row is split into segments reduced in parallel, then combined (the two-stage
shape of ViperBench/logsumexp/triton_impl.py:48-71, both stages on the GPU).
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import torch  # noqa: E402

from dslperfgap_amd import _bridge, _lib  # noqa: E402


def logsumexp(x):
    """Logsumexp reduction along the last dimension."""
    dev = _bridge.require_gpu("logsumexp", x)
    dt = _bridge.float_code(x, "logsumexp")
    if x.dim() == 0:
        x = x.reshape(1)
        out_shape = ()
    else:
        out_shape = tuple(x.shape[:-1])
    x = x.contiguous()
    cols = x.shape[-1]
    rows = _bridge.numel_prod(out_shape)
    y = _bridge.empty(x, out_shape)
    ws_bytes = _lib.logsumexp_workspace_bytes(rows, cols, dt)
    if ws_bytes:  # few long rows: split each row over several workgroups
        ws = _bridge.empty(x, (ws_bytes,), torch.uint8)
        _bridge.launch("vbh_logsumexp_fwd_ws", dev, x.data_ptr(), y.data_ptr(), rows, cols, dt,
                       dt, ws.data_ptr(), ws_bytes)
    else:
        _bridge.launch("vbh_logsumexp_fwd", dev, x.data_ptr(), y.data_ptr(), rows, cols, dt, dt)
    return y
