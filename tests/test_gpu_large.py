"""GPU parity beyond 2^31 elements (64-bit indexing).

Every kernel addresses rows and outputs with 64-bit offsets; these tensors
have 65537 x 32768 = 2,147,516,416 elements (> 2^31), so a 32-bit offset
anywhere would corrupt the last rows.  Inputs are generated on the GPU with a
seeded generator; the oracle (oracle/pytorch_impl.py) recomputes the first
and last rows on the CPU, at the loose tolerances of the reference tests
(ViperBench/test_utils.py:12-25).  The largest working set (cross entropy's
three full-size fp32 outputs) is about 35 GB of the MI355X's 288 GB.
"""
import pytest
import torch

from dslperfgap_amd.viperbench.argmax.hip_impl import argmax
from dslperfgap_amd.viperbench.cross_entropy.hip_impl import cross_entropy_fwd
from dslperfgap_amd.viperbench.layer_norm.hip_impl import layer_norm
from dslperfgap_amd.viperbench.logsumexp.hip_impl import logsumexp
from dslperfgap_amd.viperbench.mean_reduction.hip_impl import mean_reduction
from dslperfgap_amd.viperbench.rms_norm.hip_impl import rms_norm
from dslperfgap_amd.viperbench.softmax.hip_impl import softmax
from oracle import pytorch_impl as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ROWS, COLS = 65537, 32768
PICK = [0, 1, ROWS - 2, ROWS - 1]
TOL = {torch.float32: 2e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}


def _x(dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(ROWS, COLS, generator=g, device=DEV, dtype=torch.float32).to(dtype)


def _close(got, want, dtype, what):
    tol = TOL[dtype]
    g, w = got.float().cpu(), want.float()
    assert torch.allclose(g, w, atol=tol, rtol=tol), (
        f"{what}: max_err={(g - w).abs().max().item():.3e}")


@pytest.fixture(autouse=True)
def _free():
    assert ROWS * COLS > 2**31
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def test_norms_beyond_2_31_elements():
    print(f"[gpu] large norms {ROWS}x{COLS}", flush=True)
    x = _x(torch.bfloat16, 1)
    w = torch.randn(COLS, device=DEV).to(torch.bfloat16)
    b = torch.randn(COLS, device=DEV).to(torch.bfloat16)
    y = layer_norm(x, w, b)  # 1024 lanes x 4 vectors: the unguarded persistent kernel
    _close(y[PICK], ref.layer_norm(x[PICK].cpu(), w.cpu(), b.cpu()), torch.bfloat16, "layer_norm")
    del y
    z = rms_norm(x, (COLS,), w)
    _close(z[PICK], ref.rms_norm(x[PICK].cpu(), (COLS,), w.cpu()), torch.bfloat16, "rms_norm")


def test_softmax_family_beyond_2_31_elements():
    print(f"[gpu] large softmax / logsumexp {ROWS}x{COLS}", flush=True)
    x = _x(torch.float16, 2)
    y = softmax(x)
    _close(y[PICK], ref.softmax(x[PICK].cpu()), torch.float16, "softmax")
    del y, x
    xf = _x(torch.float32, 3)
    _close(logsumexp(xf)[PICK], ref.logsumexp(xf[PICK].cpu()), torch.float32, "logsumexp")


def test_reductions_beyond_2_31_elements():
    print(f"[gpu] large reductions {ROWS}x{COLS}", flush=True)
    x = _x(torch.float16, 4)
    got = argmax(x, 1)
    assert torch.equal(got[PICK].cpu(), ref.argmax(x[PICK].cpu(), 1)), "argmax rows"
    # column reduction: one lane per column walks all 65537 rows, whose offsets
    # pass 2^31 elements
    m = mean_reduction(x, 0, False, torch.float32)
    want = x[:, :64].cpu().float().mean(dim=0)
    _close(m[:64], want, torch.float32, "mean over dim 0")


def test_cross_entropy_beyond_2_31_elements():
    print(f"[gpu] large cross entropy {ROWS}x{COLS}", flush=True)
    logits = _x(torch.float32, 5)
    g = torch.Generator(device=DEV).manual_seed(6)
    labels = torch.randint(0, COLS, (ROWS,), generator=g, device=DEV)
    args = (0.0, 1.0, 0.0, -100, COLS, 0, COLS, False, False)  # one column block per row
    loss, lse, _ = cross_entropy_fwd(logits, labels, *args)
    want_loss, want_lse, _ = ref.cross_entropy_fwd(logits[PICK].cpu(), labels[PICK].cpu(), *args)
    # one block per row: row r's result sits at flat index r
    idx = torch.tensor(PICK, device=DEV)
    _close(loss.view(-1)[idx], want_loss.view(-1)[:len(PICK)], torch.float32, "loss")
    _close(lse.view(-1)[idx], want_lse.view(-1)[:len(PICK)], torch.float32, "lse")
