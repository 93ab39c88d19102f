"""GPU parity at the reference benchmark's own cases, small and large.

Every case of ``workloads.REFERENCE_CASES`` -- the shapes, dtypes and
arguments ViperBench's benchmark times for this family
(ViperBench/benchmark.py:89-97, 143-154, 187-198, 232-249, 274-291, 314-335):
LayerNorm bf16 8192^2, RMSNorm fp16 8192^2, softmax / log_softmax fp16
4096x32768, logsumexp fp32 8192x16384, cross entropy fp32 4096x32768 with
BLOCK_SIZE 1024, and argmax / max / mean over 8192x32768, plus each kernel's
"small" case.  Inputs come from the same seeded CPU generators that
``viperbench/benchmark.py`` and ``cliff_roofline.py`` time, the HIP result is
computed through the unified API (``hip_impl``), and the oracle
(oracle/pytorch_impl.py) recomputes it on the CPU.

Comparison: the reference's rule, ``torch.allclose`` on float copies with its
loose per-dtype tolerances (ViperBench/test_utils.py:12-35; fp32 2e-5, fp16
2e-3, bf16 2e-2 for atol and rtol); cross entropy on the valid block-major
positions only (cross_entropy/test.py:28-58); argmax and max indices (and max
values) exactly.
"""
import importlib

import pytest
import torch

from dslperfgap_amd import _lib
from dslperfgap_amd.workloads import REFERENCE_CASES
from oracle import pytorch_impl as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
LOOSE = {torch.float32: 2e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}
CASES = {c.key: c for c in REFERENCE_CASES}


def setup_module(module):
    _lib.lib()  # the HIP library must load on a GPU box (no fallback)


def _hip(case):
    mod = importlib.import_module(f"dslperfgap_amd.viperbench.{case.kernel}.hip_impl")
    return getattr(mod, case.fn)


def _close(got, want, what):
    assert got.device.type == "cuda", f"{what}: the HIP result must stay on the GPU"
    assert got.shape == want.shape and got.dtype == want.dtype, (
        what, got.shape, got.dtype, want.shape, want.dtype)
    tol = LOOSE[want.dtype]
    g, w = got.float().cpu(), want.float()
    if not torch.allclose(g, w, atol=tol, rtol=tol, equal_nan=True):
        err = (g - w).abs().nan_to_num(0.0).max().item()
        raise AssertionError(f"{what}: max_err={err:.3e} (atol = rtol = {tol})")


def test_every_reference_kernel_has_both_sizes():
    kernels = {c.kernel for c in REFERENCE_CASES}
    assert len(kernels) == 9
    for k in kernels:
        assert {f"{k}/small", f"{k}/large"} <= set(CASES), k


@pytest.fixture(autouse=True)
def _free():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("key", sorted(CASES))
def test_reference_case_matches_the_oracle(key):
    case = CASES[key]
    print(f"[gpu] reference case {key}: {case.desc}", flush=True)
    args = case.make()
    dev_args = tuple(a.to(DEV) if isinstance(a, torch.Tensor) else a for a in args)
    got = _hip(case)(*dev_args)
    torch.cuda.synchronize()
    want = getattr(ref, case.fn)(*args)
    if case.fn == "cross_entropy_fwd":
        logits, bs, split = args[0], int(args[8]), bool(args[10])
        n_rows, n_cols = logits.shape
        n = n_rows * -(-n_cols // bs)
        for i, (t, w) in enumerate(zip(got, want)):
            if i == 2 and split:
                continue
            assert t.shape == (n_rows, n_cols) and t.dtype == torch.float32
            _close(t.reshape(-1)[:n], w.reshape(-1)[:n], f"{key} output {i}")
    elif case.fn == "argmax":
        assert got.dtype == torch.int64
        assert torch.equal(got.cpu(), want), f"{key}: argmax indices differ"
    elif case.fn == "max_reduction":
        assert torch.equal(got[1].cpu(), want[1]), f"{key}: max indices differ"
        assert torch.equal(got[0].cpu(), want[0]), f"{key}: max values differ"
    else:
        _close(got, want, key)
