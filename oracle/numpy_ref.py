"""Float64 numpy closed forms of the normalization-family goldens.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Written independently of
oracle/pytorch_impl.py (numpy, float64, explicit formulas) so that the two can
pin each other; citations name the reference golden each formula restates.
All functions take and return numpy arrays (any float dtype in, float64 out).
"""
from __future__ import annotations

import numpy as np


def layer_norm(x, weight, bias, eps=1e-5):
    """ViperBench/layer_norm/pytorch_impl.py:12: (x - mean) / sqrt(var + eps) * w + b,
    biased variance over the trailing weight.ndim axes."""
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    axes = tuple(range(x.ndim - w.ndim, x.ndim))
    mu = x.mean(axis=axes, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=axes, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps) * w
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def rms_norm(x, normalized_shape, weight, eps=1e-5):
    """ViperBench/rms_norm/pytorch_impl.py:8-10: x / sqrt(mean(x^2) + eps) * w."""
    x = np.asarray(x, np.float64)
    nd = len(tuple(normalized_shape))
    axes = tuple(range(x.ndim - nd, x.ndim))
    ms = (x * x).mean(axis=axes, keepdims=True)
    return x / np.sqrt(ms + eps) * np.asarray(weight, np.float64).reshape(x.shape[x.ndim - nd:])


def logsumexp(x, axis=-1):
    """ViperBench/logsumexp/pytorch_impl.py:5 (torch.logsumexp): the max used as
    the shift is replaced by 0 when it is +-inf."""
    x = np.asarray(x, np.float64)
    m = np.max(x, axis=axis, keepdims=True)
    m = np.where(np.isinf(m), 0.0, m)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        s = np.exp(x - m).sum(axis=axis, keepdims=True)
        return np.squeeze(np.log(s) + m, axis=axis)


def softmax(x, axis=-1):
    """ViperBench/softmax/pytorch_impl.py:6: exp(x - max) / sum(exp(x - max))."""
    x = np.asarray(x, np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp(x - np.max(x, axis=axis, keepdims=True))
        return e / e.sum(axis=axis, keepdims=True)


def log_softmax(x, axis=-1):
    """ViperBench/log_softmax/pytorch_impl.py:8: x - max - log(sum(exp(x - max)))."""
    x = np.asarray(x, np.float64)
    m = np.max(x, axis=axis, keepdims=True)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        return (x - m) - np.log(np.exp(x - m).sum(axis=axis, keepdims=True))


def cross_entropy_rows(logits, labels, smoothing=0.0, ignored_index=-100):
    """Mean-free per-row cross entropy with label smoothing over all columns:
    (1 - s) * (lse - x_y) + s * (lse - mean(x)); 0 for ignored rows.  This is the
    single-block, no-shift case of ViperBench/cross_entropy/pytorch_impl.py:54-64."""
    x = np.asarray(logits, np.float64)
    lab = np.asarray(labels, np.int64)
    lse = logsumexp(x, axis=1)
    safe = np.clip(lab, 0, x.shape[1] - 1)
    xy = x[np.arange(x.shape[0]), safe]
    loss = (1 - smoothing) * (lse - xy) + smoothing * (lse - x.mean(axis=1))
    return np.where(lab == ignored_index, 0.0, loss)


def mean(x, axes, keepdims=False):
    """ViperBench/mean_reduction/pytorch_impl.py:8 in float64."""
    return np.asarray(x, np.float64).mean(axis=tuple(np.atleast_1d(axes)), keepdims=keepdims)


def max_argmax(x, axis, keepdims=False):
    """ViperBench/max_reduction/pytorch_impl.py:10 and argmax/pytorch_impl.py:8: the first
    position of the maximum along `axis`, where NaN counts as the largest value."""
    x = np.asarray(x, np.float64)
    nan = np.isnan(x)
    # slices holding a NaN: the first NaN; others: numpy's first-occurrence argmax
    key = np.where(nan.any(axis=axis, keepdims=True), nan.astype(np.float64), x)
    idx = np.argmax(key, axis=axis)
    vals = np.take_along_axis(x, np.expand_dims(idx, axis), axis=axis)
    if not keepdims:
        vals = np.squeeze(vals, axis=axis)
    else:
        idx = np.expand_dims(idx, axis)
    return vals, idx
