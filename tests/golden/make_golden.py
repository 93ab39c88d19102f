"""Write the golden fixtures tests/golden/<kernel>.npz.

The reference ships no golden vectors for this path (its tests compare a DSL
backend with the torch golden on unseeded CUDA inputs), so the fixtures here
are produced from seeded CPU inputs and float64 torch library routines that
restate each golden's closed form:

  layer_norm   F.layer_norm in float64      (ViperBench/layer_norm/pytorch_impl.py:12)
  rms_norm     float64 x / sqrt(mean(x^2) + eps) * w     (rms_norm/pytorch_impl.py:9-10)
  softmax      F.softmax in float64         (softmax/pytorch_impl.py:6)
  log_softmax  F.log_softmax in float64     (log_softmax/pytorch_impl.py:8)
  logsumexp    torch.logsumexp in float64   (logsumexp/pytorch_impl.py:5)
  cross_entropy  per block torch.logsumexp in float64 + the loss formulas of
               cross_entropy/pytorch_impl.py:37-76, block-major layout :80-88

Inputs are rounded to the case dtype first (bf16/fp16 values are stored as
their exact float32 values, with the dtype name alongside), so the expected
outputs are exact functions of the stored inputs.  Cases include the shapes of
the reference's own test.py files.  Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _pack(store, name, **arrays):
    for k, v in arrays.items():
        if isinstance(v, torch.Tensor):
            v = v.detach().cpu()
            v = v.float().numpy() if v.is_floating_point() else v.numpy()
        store[f"{name}__{k}"] = np.asarray(v)


def layer_norm_cases():
    s = {}
    cases = [("c16x1024_bf16", (16, 1024), "bf16"), ("c3d_2x4x1024_bf16", (2, 4, 1024), "bf16"),
             ("c16x100_f32", (16, 100), "f32"), ("c8x768_f16", (8, 768), "f16"),
             ("c2x4096_f32", (2, 4096), "f32")]
    for i, (name, shape, dt) in enumerate(cases):
        g = _gen(10 + i)
        x = torch.randn(shape, generator=g).to(DT[dt])
        w = torch.randn(shape[-1], generator=g).to(DT[dt])
        b = torch.randn(shape[-1], generator=g).to(DT[dt])
        y = F.layer_norm(x.double(), (shape[-1],), w.double(), b.double(), 1e-5)
        _pack(s, name, x=x, w=w, b=b, expected=y, dtype=np.array(dt))
    return s


def rms_norm_cases():
    s = {}
    cases = [("c4x64_f32", (4, 64), "f32"), ("c1x32_f32", (1, 32), "f32"),
             ("c32x128_f16", (32, 128), "f16"), ("c2x4096_bf16", (2, 4096), "bf16"),
             ("c8x100_f32", (8, 100), "f32")]
    for i, (name, shape, dt) in enumerate(cases):
        g = _gen(20 + i)
        x = torch.randn(shape, generator=g).to(DT[dt])
        w = torch.randn(shape[-1], generator=g).to(DT[dt])
        eps = 1e-6 if dt == "bf16" else 1e-5
        xd = x.double()
        y = xd / torch.sqrt((xd * xd).mean(dim=-1, keepdim=True) + eps) * w.double()
        _pack(s, name, x=x, w=w, expected=y, eps=np.array(eps), dtype=np.array(dt))
    return s


def softmax_family_cases():
    sm, lsm, lse = {}, {}, {}
    cases = [("c4x8_f32", (4, 8), "f32"), ("c20x100_f32", (20, 100), "f32"),
             ("c2x3x4x32_f32", (2, 3, 4, 32), "f32"), ("c128_f32", (128,), "f32"),
             ("c4x2048_f32", (4, 2048), "f32"), ("c8x256_f16", (8, 256), "f16"),
             ("c4x1000_bf16", (4, 1000), "bf16")]
    for i, (name, shape, dt) in enumerate(cases):
        g = _gen(30 + i)
        x = (3.0 * torch.randn(shape, generator=g))
        if x.numel() >= 100:
            x.view(-1)[::97] = 20.0  # large spikes, as in the measured config
        x = x.to(DT[dt])
        xd = x.double()
        _pack(sm, name, x=x, expected=F.softmax(xd, dim=-1), dtype=np.array(dt))
        _pack(lsm, name, x=x, expected=F.log_softmax(xd, dim=-1), dtype=np.array(dt))
        _pack(lse, name, x=x, expected=torch.logsumexp(xd, dim=-1), dtype=np.array(dt))
    # log_softmax over a non-last dim (4-D case of log_softmax/test.py:29)
    g = _gen(39)
    x = torch.randn(2, 8, 4, 8, generator=g)
    _pack(lsm, "dim1_2x8x4x8_f32", x=x, expected=F.log_softmax(x.double(), dim=1),
          dim=np.array(1), dtype=np.array("f32"))
    return sm, lsm, lse


def _ce_expected(logits, labels, p):
    """float64 restatement with torch.logsumexp per block."""
    L = logits.double() * p["logit_scale"]
    n_rows, n_cols = L.shape
    bs = p["BLOCK_SIZE"]
    ncb = -(-n_cols // bs)
    loss = np.zeros(n_rows * n_cols)
    lse = np.zeros(n_rows * n_cols)
    z = np.zeros(n_rows * n_cols)
    for r in range(n_rows):
        lab = int(labels[r])
        for cb in range(ncb):
            lo, hi = cb * bs, min(n_cols, (cb + 1) * bs)
            blk = L[r, lo:hi]
            l_b = float(torch.logsumexp(blk, dim=0))
            flat = cb * n_rows + r
            lse[flat] = l_b
            if lab == p["ignored_index"]:
                continue
            adj = lab - p["class_start_idx"]
            term = 0.0 if p["SPLIT"] else l_b
            ssum = float(blk.sum())
            if lo <= adj < hi:
                xy = float(L[r, adj])
                if p["HAS_SMOOTHING"]:
                    v = term - p["smoothing"] * ssum / p["total_classes"] - (1 - p["smoothing"]) * xy
                else:
                    v = term - xy
            else:
                v = p["smoothing"] * (term - ssum / p["total_classes"]) if p["HAS_SMOOTHING"] else 0.0
            if not p["SPLIT"]:
                z[flat] = p["lse_square_scale"] * l_b * l_b
                v += z[flat]
            loss[flat] = v
    return loss, lse, z


CE_PARAMS = [
    # the five configurations of ViperBench/cross_entropy/test.py:61-92 (4x8, int32 labels)
    ("ref_no_smooth_no_split_1blk", (4, 8), "i32",
     dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1,
          total_classes=10, class_start_idx=0, BLOCK_SIZE=8, HAS_SMOOTHING=False, SPLIT=False)),
    ("ref_smooth_no_split_1blk", (4, 8), "i32",
     dict(smoothing=0.1, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1,
          total_classes=10, class_start_idx=0, BLOCK_SIZE=8, HAS_SMOOTHING=True, SPLIT=False)),
    ("ref_smooth_split_1blk", (4, 8), "i32",
     dict(smoothing=0.1, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1,
          total_classes=10, class_start_idx=0, BLOCK_SIZE=8, HAS_SMOOTHING=True, SPLIT=True)),
    ("ref_no_smooth_no_split_2blk", (4, 8), "i32",
     dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1,
          total_classes=10, class_start_idx=0, BLOCK_SIZE=4, HAS_SMOOTHING=False, SPLIT=False)),
    ("ref_logit_scale_2blk", (4, 8), "i32",
     dict(smoothing=0.0, logit_scale=0.5, lse_square_scale=0.05, ignored_index=-1,
          total_classes=10, class_start_idx=0, BLOCK_SIZE=4, HAS_SMOOTHING=False, SPLIT=False)),
    # wider rows, ragged last block, ignored rows, shifted class range, int64 labels
    ("ragged_16x1000_bs256_ignored", (16, 1000), "i64",
     dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0, ignored_index=-100,
          total_classes=1000, class_start_idx=0, BLOCK_SIZE=256, HAS_SMOOTHING=False, SPLIT=False)),
    ("shifted_8x500_split_smooth", (8, 500), "i64",
     dict(smoothing=0.2, logit_scale=1.0, lse_square_scale=0.0, ignored_index=-100,
          total_classes=2000, class_start_idx=500, BLOCK_SIZE=128, HAS_SMOOTHING=True, SPLIT=True)),
    ("one_block_4x1024_zloss", (4, 1024), "i32",
     dict(smoothing=0.0, logit_scale=2.0, lse_square_scale=1e-4, ignored_index=-100,
          total_classes=1024, class_start_idx=0, BLOCK_SIZE=1024, HAS_SMOOTHING=False, SPLIT=False)),
]


def ce_cases():
    s = {}
    for i, (name, (n_rows, n_cols), ldt, p) in enumerate(CE_PARAMS):
        g = _gen(50 + i)
        logits = torch.randn(n_rows, n_cols, generator=g)
        lo = -p["class_start_idx"] if p["class_start_idx"] else 0
        hi = p["total_classes"] if p["class_start_idx"] else n_cols
        labels = torch.randint(max(lo, 0), hi, (n_rows,), generator=g)
        if "ignored" in name:
            labels[::7] = p["ignored_index"]
        labels = labels.to(torch.int32 if ldt == "i32" else torch.int64)
        loss, lse, z = _ce_expected(logits, labels, p)
        _pack(s, name, logits=logits, labels=labels, loss=loss, lse=lse, z_loss=z,
              params=np.array(json.dumps(p)))
    return s


def main():
    sm, lsm, lse = softmax_family_cases()
    files = {"layer_norm": layer_norm_cases(), "rms_norm": rms_norm_cases(), "softmax": sm,
             "log_softmax": lsm, "logsumexp": lse, "cross_entropy": ce_cases()}
    for kernel, arrays in files.items():
        path = OUT / f"{kernel}.npz"
        np.savez_compressed(path, **arrays)
        print(f"{path.name}: {len(arrays)} arrays, {path.stat().st_size} bytes")


if __name__ == "__main__":
    main()
