"""The reference test.py case lists, run through the run_test-format recorder.

Each kernel's cases are those of ViperBench/<kernel>/test.py (names, shapes,
dtypes, arguments, loose_tol and compare function), with inputs drawn from a
seeded CPU generator instead of unseeded ``torch.randn(..., device='cuda')``.
``dslperfgap_amd.viperbench.test_utils.run_test`` runs the oracle (the
restated golden, on the CPU) and the hip impl (on the GPU) on each case and
writes ``<kernel>_hip.json`` -- ``{"kernel", "overall", "test_cases"}`` with
each case's status, max_err and time_ms, as ViperBench/results/<kernel>.json
-- into ``$VBH_RECORDS_DIR`` (default: dslperfgap_amd/viperbench/results).
Every record must come out PASS.
"""
import os
from pathlib import Path

import pytest
import torch

from dslperfgap_amd.viperbench import test_utils as tu
from oracle import pytorch_impl as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
RECORDS = Path(os.environ.get("VBH_RECORDS_DIR", str(tu.RESULTS_DIR)))


def _gen(kernel):
    return torch.Generator().manual_seed(9000 + sum(map(ord, kernel)))


def _randn(g, *shape, dtype=torch.float32):
    return torch.randn(*shape, generator=g).to(dtype)


def _to_dev(inputs):
    return tuple(t.to(DEV) if isinstance(t, torch.Tensor) else t for t in inputs)


def _hip(kernel, fn=None):
    import importlib

    mod = importlib.import_module(f"dslperfgap_amd.viperbench.{kernel}.hip_impl")
    return getattr(mod, fn or kernel)


def _layer_norm_cases():
    g = _gen("layer_norm")  # layer_norm/test.py:12-26

    def case(name, shape, d, dtype=torch.bfloat16):
        return {"name": name, "dtype": dtype, "inputs": (_randn(g, *shape, dtype=dtype),
                                                         _randn(g, d, dtype=dtype),
                                                         _randn(g, d, dtype=dtype))}
    return [case("128x1024_bf16", (128, 1024), 1024), case("256x2048_bf16", (256, 2048), 2048),
            case("64x4096_bf16", (64, 4096), 4096), case("512x1024_bf16", (512, 1024), 1024),
            case("3d_4x32x1024_bf16", (4, 32, 1024), 1024),
            case("3d_2x8x2048_bf16", (2, 8, 2048), 2048)]


def _rms_norm_cases():
    g = _gen("rms_norm")  # rms_norm/test.py:12-15, 30-36

    def case(name, b, f, dtype):
        return {"name": name, "dtype": dtype,
                "inputs": (_randn(g, b, f, dtype=dtype), (f,), _randn(g, f, dtype=dtype))}
    return [case("small_fp32", 4, 64, torch.float32), case("medium_fp32", 32, 128, torch.float32),
            case("large_fp32", 128, 512, torch.float32), case("edge_fp32", 1, 32, torch.float32),
            case("small_fp16", 32, 128, torch.float16)]


def _x_cases(kernel, spec):
    g = _gen(kernel)
    return [{"name": n, "dtype": dt, "inputs": (_randn(g, *shape, dtype=dt),)}
            for n, shape, dt in spec]


F32, F16 = torch.float32, torch.float16
SOFTMAX = [("small_2d", (4, 8), F32), ("medium_2d", (128, 512), F32),  # softmax/test.py:11-28
           ("large_cols", (64, 4096), F32), ("wide", (16, 2048), F32), ("square", (100, 100), F32),
           ("3d_tensor", (4, 8, 64), F32), ("4d_tensor", (2, 3, 4, 32), F32),
           ("1d_tensor", (128,), F32)]
LOG_SOFTMAX = [("small_fp32", (4, 64), F32), ("medium_fp32", (32, 256), F32),  # :25-31
               ("large_fp32", (128, 1024), F32), ("4d_fp32", (2, 8, 128, 64), F32),
               ("small_fp16", (32, 256), F16)]
LOGSUMEXP = [("small_2d", (4, 64), F32), ("medium_2d", (32, 256), F32),  # logsumexp/test.py:10-25
             ("large_2d", (128, 1024), F32), ("wide_2d", (8, 4096), F32),
             ("3d_tensor", (4, 8, 64), F32), ("4d_tensor", (2, 3, 4, 32), F32),
             ("1d_tensor", (128,), F32)]


def _red_cases(kernel, spec):
    g = _gen(kernel)
    return [{"name": n, "dtype": F32, "inputs": (_randn(g, *shape),) + tuple(rest)}
            for n, shape, rest in spec]


MEAN = [("2D_dim0", (64, 128), (0,)), ("2D_dim1_keepdim", (64, 128), (1, True)),  # :12-33
        ("4D_multi_dim", (2, 3, 4, 5), ([1, 2],)), ("3D_dim2", (8, 16, 32), (2,))]
MAX = [("2D_dim0", (128, 256), (0,)), ("2D_dim1", (256, 128), (1,)),  # max_reduction/test.py:13-38
       ("3D_dim2", (32, 64, 128), (2,)), ("2D_dim1_keepdim", (64, 256), (1, True)),
       ("3D_neg_dim", (16, 32, 64), (-1,))]
ARGMAX = [("2D_dim0", (128, 256), (0,)), ("2D_dim1", (256, 128), (1,)),  # argmax/test.py:13-33
          ("3D_dim2", (32, 64, 128), (2,)), ("3D_dim1_keepdim", (16, 32, 64), (1, True))]


def compare_max(r, t, dtype, loose):
    """max_reduction/test.py:41-49: values within tolerance, indices equal."""
    vp, ve = tu.default_compare(r[0], t[0], dtype, loose)
    ip = torch.equal(r[1], t[1].cpu())
    ie = 0.0 if ip else (r[1].float() - t[1].cpu().float()).abs().max().item()
    return vp and ip, max(ve, ie)


def compare_indices(r, t, dtype, loose):
    """argmax/test.py:36-40: int64 indices exactly."""
    p = torch.equal(r, t.cpu())
    return p, 0.0 if p else (r.float() - t.cpu().float()).abs().max().item()


CE_CONFIGS = [  # cross_entropy/test.py:61-92
    ("no_smooth_no_split_1blk", dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.1,
                                     BLOCK_SIZE=8, HAS_SMOOTHING=False, SPLIT=False)),
    ("smooth_no_split_1blk", dict(smoothing=0.1, logit_scale=1.0, lse_square_scale=0.1,
                                  BLOCK_SIZE=8, HAS_SMOOTHING=True, SPLIT=False)),
    ("smooth_split_1blk", dict(smoothing=0.1, logit_scale=1.0, lse_square_scale=0.1,
                               BLOCK_SIZE=8, HAS_SMOOTHING=True, SPLIT=True)),
    ("no_smooth_no_split_2blk", dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.1,
                                     BLOCK_SIZE=4, HAS_SMOOTHING=False, SPLIT=False)),
    ("logit_scale_2blk", dict(smoothing=0.0, logit_scale=0.5, lse_square_scale=0.05,
                              BLOCK_SIZE=4, HAS_SMOOTHING=False, SPLIT=False)),
]


def _ce_compare(r, t, dtype, loose, kw):
    """cross_entropy/test.py:28-58: the valid block-major positions only,
    z_loss skipped with SPLIT, at the loose tolerance."""
    n_rows, n_cols = kw["logits"].shape
    n = n_rows * -(-n_cols // kw["BLOCK_SIZE"])
    keep = [k for k in range(3) if not (k == 2 and kw["SPLIT"])]
    return tu.default_compare(tuple(r[k].reshape(-1)[:n] for k in keep),
                              tuple(t[k].reshape(-1)[:n] for k in keep), dtype, True)


def _ce_cases():
    g = _gen("cross_entropy")  # cross_entropy/test.py:13-17: 4 x 8 logits, int32 labels
    logits = _randn(g, 4, 8)
    labels = torch.randint(0, 8, (4,), generator=g, dtype=torch.int32)
    out = []
    for name, p in CE_CONFIGS:
        kw = dict(logits=logits, labels=labels, ignored_index=-1, total_classes=10,
                  class_start_idx=0, **p)
        out.append({"name": name, "dtype": F32, "inputs": kw,
                    "compare": lambda r, t, d, lo, kw=kw: _ce_compare(r, t, d, lo, kw)})
    return out


def _ce_to_dev(inputs):
    return {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in inputs.items()}


RECORDED = {
    # kernel: (cases, oracle fn, hip fn, loose_tol, compare_fn, to_device)
    "layer_norm": (_layer_norm_cases, ref.layer_norm, _hip("layer_norm"), True, None, _to_dev),
    "rms_norm": (_rms_norm_cases, ref.rms_norm, _hip("rms_norm"), True, None, _to_dev),
    "softmax": (lambda: _x_cases("softmax", SOFTMAX), ref.softmax, _hip("softmax"), True, None,
                _to_dev),
    "log_softmax": (lambda: _x_cases("log_softmax", LOG_SOFTMAX),
                    lambda x: ref.log_softmax(x, dim=-1),
                    lambda x: _hip("log_softmax")(x, dim=-1), True, None, _to_dev),
    "logsumexp": (lambda: _x_cases("logsumexp", LOGSUMEXP), ref.logsumexp, _hip("logsumexp"),
                  True, None, _to_dev),
    "cross_entropy": (_ce_cases, ref.cross_entropy_fwd, _hip("cross_entropy", "cross_entropy_fwd"),
                      True, None, _ce_to_dev),
    "mean_reduction": (lambda: _red_cases("mean_reduction", MEAN), ref.mean_reduction,
                       _hip("mean_reduction"), True, None, _to_dev),
    "max_reduction": (lambda: _red_cases("max_reduction", MAX), ref.max_reduction,
                      _hip("max_reduction"), False, compare_max, _to_dev),
    "argmax": (lambda: _red_cases("argmax", ARGMAX), ref.argmax, _hip("argmax"), False,
               compare_indices, _to_dev),
}


@pytest.mark.parametrize("kernel", sorted(RECORDED))
def test_reference_cases_recorded(kernel):
    make, oracle_fn, hip_fn, loose, cmp, to_dev = RECORDED[kernel]
    print(f"[gpu] run_test record {kernel}", flush=True)
    ok, rec = tu.run_test(kernel, make(), oracle_fn, hip_fn, loose_tol=loose, compare_fn=cmp,
                          results_dir=RECORDS, to_device=to_dev)
    assert (RECORDS / f"{kernel}_hip.json").exists()
    bad = [c for c in rec["test_cases"] if c["status"] != "PASS"]
    assert ok and rec["overall"] == "PASS", bad
