"""ViperBench/cross_entropy - HIP backend.

Unified API of ViperBench/cross_entropy/pytorch_impl.py:4-90 / 93-141
(flash-attn style column-blocked cross entropy):

``cross_entropy_fwd(logits, labels, smoothing, logit_scale, lse_square_scale,
ignored_index, total_classes, class_start_idx, BLOCK_SIZE, HAS_SMOOTHING, SPLIT)``
returns ``(loss, lse, z_loss)``, three fp32 ``[n_rows, n_cols]`` tensors holding
the per-(row, column block) results at flat index ``cb * n_rows + row``.

Like the Triton backend (ViperBench/cross_entropy/triton_impl.py:128-130) the
outputs are allocated with ``torch.empty`` and only the ``n_rows * ncb`` valid
positions are written; the golden additionally zero-fills the tail, which
ViperBench's own CE test never reads (cross_entropy/test.py:28-58).  With
SPLIT the z_loss positions are written as 0, as in the golden.

``cross_entropy_bwd(dloss, logits, lse, labels, ...)`` returns dlogits shaped
like logits; ``lse`` is read at flat index ``row`` (a per-row vector, or the
forward's lse buffer when there is one column block).
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import torch  # noqa: E402

from dslperfgap_amd import _bridge, _lib  # noqa: E402


def _labels(labels, n_rows, what):
    if labels.dim() != 1 or labels.shape[0] != n_rows:
        raise ValueError(f"{what}: labels must have shape [{n_rows}], got {list(labels.shape)}")
    if labels.dtype not in _bridge.LABEL_CODES:
        if labels.dtype.is_floating_point or labels.dtype == torch.bool:
            raise TypeError(f"{what}: labels must be an integer tensor, got {labels.dtype}")
        labels = labels.to(torch.int64)  # the golden's labels.to(torch.int64)
    return labels.contiguous()


def _logits(logits, what):
    if logits.dim() != 2:
        raise ValueError(f"{what}: logits must be 2-D [n_rows, n_cols], got {list(logits.shape)}")
    st = logits.stride()
    if st[1] != 1 or st[0] < logits.shape[1]:
        logits = logits.contiguous()
    return logits


def cross_entropy_fwd(
    logits, labels, smoothing, logit_scale, lse_square_scale,
    ignored_index, total_classes, class_start_idx, BLOCK_SIZE, HAS_SMOOTHING, SPLIT
):
    """Column-blocked CE forward; see the module docstring for the layout."""
    what = "cross_entropy_fwd"
    dev = _bridge.require_gpu(what, logits, labels)
    if int(BLOCK_SIZE) <= 0:
        raise ValueError(f"{what}: BLOCK_SIZE must be positive, got {BLOCK_SIZE}")
    logits = _logits(logits, what)
    n_rows, n_cols = logits.shape
    labels = _labels(labels, n_rows, what)
    dt = _bridge.float_code(logits, what)
    loss = _bridge.empty(logits, (n_rows, n_cols), torch.float32)
    lse = _bridge.empty(logits, (n_rows, n_cols), torch.float32)
    z_loss = _bridge.empty(logits, (n_rows, n_cols), torch.float32)
    row_stride = logits.stride(0) if n_rows > 1 else n_cols
    args = (logits.data_ptr(), labels.data_ptr(), dt, _bridge.LABEL_CODES[labels.dtype],
            loss.data_ptr(), lse.data_ptr(), z_loss.data_ptr(), n_rows, n_cols, row_stride,
            float(smoothing), float(logit_scale), float(lse_square_scale), int(ignored_index),
            int(total_classes), int(class_start_idx), int(BLOCK_SIZE), int(bool(HAS_SMOOTHING)),
            int(bool(SPLIT)))
    ws_bytes = _lib.cross_entropy_workspace_bytes(n_rows, n_cols, int(BLOCK_SIZE), dt)
    if ws_bytes:  # few long rows in one column block: split each row over workgroups
        ws = _bridge.empty(logits, (ws_bytes,), torch.uint8)
        _bridge.launch("vbh_cross_entropy_fwd_ws", dev, *args, ws.data_ptr(), ws_bytes)
    else:
        _bridge.launch("vbh_cross_entropy_fwd", dev, *args)
    return loss, lse, z_loss


def cross_entropy_bwd(
    dloss, logits, lse, labels, smoothing, logit_scale, lse_square_scale,
    ignored_index, total_classes, class_start_idx, BLOCK_SIZE, HAS_SMOOTHING
):
    """dlogits = dloss * logit_scale * (softmax(+ z-loss term) - smoothed one-hot)."""
    what = "cross_entropy_bwd"
    dev = _bridge.require_gpu(what, dloss, logits, lse, labels)
    if int(BLOCK_SIZE) <= 0:
        raise ValueError(f"{what}: BLOCK_SIZE must be positive, got {BLOCK_SIZE}")
    logits = _logits(logits, what)
    n_rows, n_cols = logits.shape
    labels = _labels(labels, n_rows, what)
    dt = _bridge.float_code(logits, what)
    dl = dloss.reshape(-1).to(torch.float32)
    if dl.numel() < n_rows:
        raise ValueError(f"{what}: dloss has {dl.numel()} elements for {n_rows} rows")
    lse_flat = lse.reshape(-1).to(torch.float32).contiguous()
    if lse_flat.numel() < n_rows:
        raise ValueError(f"{what}: lse has {lse_flat.numel()} elements for {n_rows} rows")
    dlogits = _bridge.empty(logits, (n_rows, n_cols))
    _bridge.launch("vbh_cross_entropy_bwd", dev, _bridge.ptr(dl), _bridge.ptr(logits),
                   _bridge.ptr(lse_flat), _bridge.ptr(labels), _bridge.ptr(dlogits), dt,
                   _bridge.LABEL_CODES[labels.dtype], n_rows, n_cols,
                   logits.stride(0) if n_rows > 1 else n_cols, n_cols,
                   dl.stride(0) if dl.numel() > 1 else 1, float(smoothing),
                   float(logit_scale), float(lse_square_scale), int(ignored_index),
                   int(total_classes), int(class_start_idx), int(bool(HAS_SMOOTHING)))
    return dlogits


def loss_mean(loss, n_rows):
    """The scalar loss of a mean-reduced cross entropy: the mean of the first
    ``n_rows`` flat positions of the forward's ``loss`` -- with one column
    block per row, the per-row losses (``loss.view(-1)[:n_rows].mean()``, the
    scalar of BASELINE.json's C4 config).  Computed on the GPU by the library's
    mean reduction (vbh_reduce_fwd: fp32 row sum, then / n_rows); returns a 0-d
    fp32 tensor on loss's device."""
    what = "cross_entropy loss_mean"
    dev = _bridge.require_gpu(what, loss)
    n_rows = int(n_rows)
    flat = loss.reshape(-1)
    if loss.dtype != torch.float32:
        raise TypeError(f"{what}: loss must be fp32, got {loss.dtype}")
    if not 0 < n_rows <= flat.numel():
        raise ValueError(f"{what}: n_rows {n_rows} outside 1..{flat.numel()}")
    flat = flat[:n_rows].contiguous()
    out = _bridge.empty(flat, ())
    _bridge.launch("vbh_reduce_fwd", dev, flat.data_ptr(), out.data_ptr(), None, 1, n_rows, 1,
                   _lib.F32, _lib.F32, _lib.REDUCE_MEAN)
    return out
