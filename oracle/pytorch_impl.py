"""CPU torch restatement of ViperBench's normalization-family goldens.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the checker that GPU
results are compared against, and the timed path of bench.py's cpu_baseline.

Each function keeps the reference's unified-API signature and semantics; the
reference file:line it follows is cited in its docstring.  Inputs may live on
any device; the computation happens where the inputs are (tests pass CPU
tensors).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def layer_norm(x, weight, bias, eps=1e-5):
    """ViperBench/layer_norm/pytorch_impl.py:5-12.

    F.layer_norm over the trailing ``weight.shape`` dims; eps other than 1e-5
    raises ValueError, as the golden does.
    """
    if eps != 1e-5:
        raise ValueError(f"Only eps=1e-5 is supported (got {eps}). "
                         "The Triton kernel hardcodes eps=1e-5.")
    return F.layer_norm(x, tuple(weight.shape), weight, bias, eps)


def rms_norm(x, normalized_shape, weight, eps=1e-5):
    """ViperBench/rms_norm/pytorch_impl.py:3-10.

    Mean of squares over the last ``len(normalized_shape)`` dims in fp32,
    ``x.float() / sqrt(ms + eps) * weight.float()``, cast back to x's dtype.
    """
    nd = len(tuple(normalized_shape))
    axes = tuple(range(x.dim() - nd, x.dim()))
    xf = x.float()
    denom = torch.sqrt((xf * xf).mean(dim=axes, keepdim=True) + eps)
    return ((xf / denom) * weight.float()).to(x.dtype)


def softmax(x):
    """ViperBench/softmax/pytorch_impl.py:4-6: F.softmax over the last dim."""
    return F.softmax(x, dim=-1)


def log_softmax(x, dim=-1, dtype=None):
    """ViperBench/log_softmax/pytorch_impl.py:4-8: F.log_softmax(x, dim, dtype)."""
    return F.log_softmax(x, dim=dim, dtype=dtype)


def logsumexp(x):
    """ViperBench/logsumexp/pytorch_impl.py:3-5: torch.logsumexp over the last dim."""
    return torch.logsumexp(x, dim=-1)


def _block_view(logits, logit_scale, block):
    """Scaled fp32 logits padded with -inf to whole blocks: [rows, nblocks, block]."""
    rows, cols = logits.shape
    nb = -(-cols // block)
    padded = torch.full((rows, nb * block), float("-inf"), dtype=torch.float32,
                        device=logits.device)
    padded[:, :cols] = logits.float() * logit_scale
    return padded.view(rows, nb, block), nb


def _to_flat_layout(per_block, rows, cols):
    """[rows, nblocks] -> the kernel layout: flat[cb * rows + r], zero tail, [rows, cols]."""
    flat = per_block.t().reshape(-1)
    out = torch.zeros(rows * cols, dtype=torch.float32, device=per_block.device)
    n = min(flat.numel(), out.numel())
    out[:n] = flat[:n]
    return out.view(rows, cols)


def cross_entropy_fwd(logits, labels, smoothing, logit_scale, lse_square_scale,
                      ignored_index, total_classes, class_start_idx, BLOCK_SIZE,
                      HAS_SMOOTHING, SPLIT):
    """ViperBench/cross_entropy/pytorch_impl.py:4-90 (vectorized golden).

    Per (row, column block cb): lse = log(sum(exp(L - max))) + max over the
    block's scaled logits (padding = -inf, :29-35); the label counts for the
    block holding ``label - class_start_idx`` (bounds test :43-46); loss with or
    without smoothing (:54-64), plus z = lse_square_scale * lse^2 unless SPLIT
    (:66-70); ignored rows give loss = z = 0 (:74-76).  Results are stored at
    flat index cb * n_rows + row of zero-filled [n_rows, n_cols] buffers (:80-88).
    """
    rows, cols = logits.shape
    Lb, nb = _block_view(logits, logit_scale, BLOCK_SIZE)
    bmax = Lb.max(dim=2).values
    lse = torch.log(torch.exp(Lb - bmax.unsqueeze(2)).sum(dim=2)) + bmax

    lab = labels.to(torch.int64)
    shifted = lab - class_start_idx
    keep = lab != ignored_index
    starts = torch.arange(nb, device=logits.device) * BLOCK_SIZE
    ends = torch.clamp(starts + BLOCK_SIZE, max=cols)
    hit = (shifted[:, None] >= starts[None, :]) & (shifted[:, None] < ends[None, :])

    gather_at = shifted.clamp(0, cols - 1)
    picked = logits.gather(1, gather_at[:, None]).float()[:, 0] * logit_scale
    base = torch.zeros_like(lse) if SPLIT else lse

    if HAS_SMOOTHING:
        valid = (torch.arange(nb * BLOCK_SIZE, device=logits.device) < cols).view(1, nb, BLOCK_SIZE)
        blk_sum = torch.where(valid, Lb, torch.zeros_like(Lb)).sum(dim=2)
        on = base - smoothing * blk_sum / total_classes - (1 - smoothing) * picked[:, None]
        off = smoothing * (base - blk_sum / total_classes)
        loss = torch.where(hit, on, off)
    else:
        loss = torch.where(hit, base - picked[:, None], torch.zeros_like(lse))

    if SPLIT:
        z = torch.zeros_like(lse)
    else:
        z = lse_square_scale * lse * lse
        loss = loss + z

    loss = torch.where(keep[:, None], loss, torch.zeros_like(loss))
    z = torch.where(keep[:, None], z, torch.zeros_like(z))
    return (_to_flat_layout(loss, rows, cols), _to_flat_layout(lse, rows, cols),
            _to_flat_layout(z, rows, cols))


def cross_entropy_bwd(dloss, logits, lse, labels, smoothing, logit_scale, lse_square_scale,
                      ignored_index, total_classes, class_start_idx, BLOCK_SIZE, HAS_SMOOTHING):
    """ViperBench/cross_entropy/pytorch_impl.py:93-141, vectorized over rows.

    dlogits[r, c] = (dl_r * logit_scale) * q, where dl_r = dloss[r] (0 for an
    ignored row), p = exp(logit_scale * x - lse[r]), q = p + 2 * lse_square_scale
    * lse[r] * p, minus (1 - smoothing) (or 1) at the shifted label column, minus
    smoothing / total_classes everywhere when smoothing.  ``lse`` is read per row
    (flat index r).
    """
    rows, cols = logits.shape
    lab = labels.to(torch.int64)
    lse_r = lse.reshape(-1)[:rows].float()
    dl = dloss.reshape(-1)[:rows].double()
    dl = torch.where(lab != ignored_index, dl, torch.zeros_like(dl))
    scale = (dl * logit_scale).float()                       # Python-double product
    p = torch.exp(logits.float() * logit_scale - lse_r[:, None])
    p = p + (2.0 * lse_square_scale) * lse_r[:, None] * p
    col = torch.arange(cols, device=logits.device)[None, :]
    at_label = col == (lab - class_start_idx)[:, None]
    if HAS_SMOOTHING:
        p = torch.where(at_label, p - (1 - smoothing), p) - smoothing / total_classes
    else:
        p = torch.where(at_label, p - 1.0, p)
    return (scale[:, None] * p).to(logits.dtype)


def mean_reduction(input_tensor, dim, keepdim=False, dtype=None):
    """ViperBench/mean_reduction/pytorch_impl.py:4-8: torch.mean(x, dim, keepdim, dtype)."""
    return torch.mean(input_tensor, dim, keepdim=keepdim, dtype=dtype)


def max_reduction(input, dim, keepdim=False):
    """ViperBench/max_reduction/pytorch_impl.py:4-11: torch.max along `dim` -> (values, indices)."""
    if not isinstance(input, torch.Tensor):
        raise TypeError('The input must be a torch.Tensor.')
    values, indices = torch.max(input, dim, keepdim=keepdim)
    return (values, indices)


def argmax(input_tensor, dim, keepdim=False):
    """ViperBench/argmax/pytorch_impl.py:4-8: torch.argmax(x, dim=dim, keepdim=keepdim)."""
    return torch.argmax(input_tensor, dim=dim, keepdim=keepdim)
