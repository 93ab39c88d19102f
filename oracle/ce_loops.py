"""Brute-force per-program loops for the column-blocked cross entropy.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  One Python iteration per
(row, column block) "program", following the program body of
ViperBench/cross_entropy/triton_impl.py:33-75 (forward) and :98-120 (backward),
in float64 with plain ``math`` functions.  Meant for tiny inputs (a few
thousand elements); returns flat Python lists in the kernel's block-major
layout (forward) or a nested list (backward).
"""
from __future__ import annotations

import math


def cross_entropy_fwd(logits, labels, smoothing, logit_scale, lse_square_scale, ignored_index,
                      total_classes, class_start_idx, block_size, has_smoothing, split):
    """logits: list of rows (floats); labels: list of ints.  Returns
    (loss, lse, z_loss) as dicts {flat_index: value} for flat = cb * n_rows + row."""
    n_rows = len(logits)
    n_cols = len(logits[0]) if n_rows else 0
    ncb = -(-n_cols // block_size)
    loss, lse_out, z_out = {}, {}, {}
    for row in range(n_rows):
        for cb in range(ncb):
            lo, hi = cb * block_size, min(n_cols, (cb + 1) * block_size)
            vals = [logits[row][c] * logit_scale for c in range(lo, hi)]
            m = max(vals)
            lse = math.log(sum(math.exp(v - m) for v in vals)) + m
            flat = cb * n_rows + row
            lse_out[flat] = lse
            label = labels[row]
            if label == ignored_index:
                loss[flat], z_out[flat] = 0.0, 0.0
                continue
            adj = label - class_start_idx
            term = 0.0 if split else lse
            if lo <= adj < hi:
                xy = logits[row][adj] * logit_scale
                if has_smoothing:
                    l = term - smoothing * sum(vals) / total_classes - (1 - smoothing) * xy
                else:
                    l = term - xy
            else:
                l = smoothing * (term - sum(vals) / total_classes) if has_smoothing else 0.0
            if split:
                z = 0.0
            else:
                z = lse_square_scale * lse * lse
                l += z
            loss[flat], z_out[flat] = l, z
    return loss, lse_out, z_out


def cross_entropy_bwd(dloss, logits, lse, labels, smoothing, logit_scale, lse_square_scale,
                      ignored_index, total_classes, class_start_idx, has_smoothing):
    """dlogits as a list of rows; lse[r] is the per-row log-sum-exp."""
    out = []
    for row, xs in enumerate(logits):
        label = labels[row]
        dl = dloss[row] if label != ignored_index else 0.0
        adj = label - class_start_idx
        r = []
        for c, x in enumerate(xs):
            p = math.exp(x * logit_scale - lse[row])
            p += 2.0 * lse_square_scale * lse[row] * p
            if c == adj:
                p -= (1 - smoothing) if has_smoothing else 1.0
            if has_smoothing:
                p -= smoothing / total_classes
            r.append(dl * logit_scale * p)
        out.append(r)
    return out
