"""GPU parity of the exp-based kernels on rows whose maximum is far from 0.

The register-resident softmax / log_softmax / logsumexp / cross-entropy
kernels compute exp(x - m) as 2^(x * log2 e - m * log2 e) with m * log2 e
rounded once per row.  That rounding grows with |m| (at 1e10 it scales every
exp by 2^-440; above 2.36e38 the product overflows), so rows whose finite
shift exceeds 2^24 take exp(x - m) on a subtract.  These cases put such rows
next to ordinary ones in one launch (short rows share a wave, so both forms
run side by side), over every launch path: rows of one vector or less, rows
not a multiple of the vector, register-resident rows, the streaming kernels,
the split softmax / logsumexp / cross-entropy, and the tiled backward.

Row kinds, per dtype: the dtype's most negative finite value everywhere (the
usual attention-mask fill: softmax 1/n, logsumexp min + log n), N(0,1) values
with one entry at 3e38 (fp16: its largest finite value), values around -3e38,
around 1e10 and -1e12 (the FMA form's residual would underflow or overflow
every exp), around 3e7 with spacings of a few units (the subtract form gives
exps that are neither 0 nor 1), and ordinary N(0,1) and 1e4 * N(0,1) rows.
The expectation is the oracle (the restated reference golden, torch on the
CPU) on the same inputs; tolerances are the reference's loose per-dtype set
(ViperBench/test_utils.py:12-25).
"""
import pytest
import torch

from dslperfgap_amd.viperbench.cross_entropy.hip_impl import cross_entropy_bwd, cross_entropy_fwd
from dslperfgap_amd.viperbench.log_softmax.hip_impl import log_softmax
from dslperfgap_amd.viperbench.logsumexp.hip_impl import logsumexp
from dslperfgap_amd.viperbench.softmax.hip_impl import softmax
from oracle import pytorch_impl as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
LOOSE = {torch.float32: 2e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
# one vector or less, not a multiple of the vector, register-resident,
# C3's width, a C4-like width, the streaming kernels, the split path
WIDTHS = [8, 100, 1000, 1024, 4096, 32000, 70000, 131072]


def _rows(dtype, cols, seed):
    """Eight rows, one per kind, in `dtype`."""
    g = torch.Generator().manual_seed(seed)
    fin = torch.finfo(dtype)
    n = torch.randn(8, cols, generator=g, dtype=torch.float64)
    steps = torch.randint(-10, 1, (8, cols), generator=g).double()
    x = torch.empty(8, cols, dtype=torch.float64)
    x[0] = fin.min
    x[1] = n[1]
    x[1, cols // 3] = 3e38 if dtype != torch.float16 else fin.max
    if dtype == torch.float16:
        # fp16 has no values beyond 65504: its extremes, and ordinary spreads.
        # Its extreme rows are spread over four values (ulp 32 there): torch's
        # CPU fp16 log_softmax / logsumexp keep the row sum in fp16, so a row
        # of more than 65504 equal values overflows it to -inf / inf, where
        # the reference's CUDA golden sums in fp32.
        x[0] = fin.min + 32.0 * steps[0].abs().remainder(4)
        x[2] = -60000.0 + 100.0 * steps[2]
        x[3] = fin.max - 32.0 * steps[3].abs().remainder(4)
        x[4] = 1000.0 + 2.0 * steps[4]
        x[6] = -30000.0 + 50.0 * steps[6]
    else:
        x[2] = -3.0e38 * (1.0 + 0.05 * steps[2].abs())
        x[3] = 1e10 + 1024.0 * steps[3]
        # spacing 2 is exact in fp32 around 3e7; bf16 keeps 8 bits there
        x[4] = 3e7 + (2.0 if dtype == torch.float32 else 131072.0) * steps[4]
        x[6] = -1e12 + 65536.0 * steps[6]
    x[5] = n[5]
    x[7] = 1e4 * n[7]
    return x.to(dtype)


def _close(got, want, dtype, what):
    assert got.device.type == "cuda", what
    assert got.shape == want.shape and got.dtype == want.dtype, (what, got.shape, want.shape)
    tol = LOOSE[dtype]
    g, w = got.float().cpu(), want.float()
    ok = torch.allclose(g, w, atol=tol, rtol=tol, equal_nan=True)
    if not ok:
        bad = ~torch.isclose(g, w, atol=tol, rtol=tol, equal_nan=True)
        rows = sorted(set(torch.nonzero(bad.reshape(bad.shape[0], -1))[:, 0].tolist()))
        err = (g - w).abs().nan_to_num(0.0).max().item()
        raise AssertionError(f"{what}: rows {rows} differ, max_err={err:.3e} tol={tol}")


@pytest.mark.parametrize("cols", WIDTHS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_softmax_family_far_shifts(cols, dtype):
    print(f"[gpu] far shifts softmax family {dtype} 8x{cols}", flush=True)
    x = _rows(dtype, cols, 7000 + cols)
    xd = x.to(DEV)
    want_sm = ref.softmax(x)
    # the kinds' closed forms pin the oracle itself: a fill row is uniform, a
    # single far spike takes all the mass
    if dtype != torch.float16:
        assert torch.allclose(want_sm[0].double(),
                              torch.full((cols,), 1.0 / cols, dtype=torch.float64),
                              rtol=LOOSE[dtype], atol=0)
    assert want_sm[1, cols // 3].item() == 1.0 or dtype == torch.float16
    _close(softmax(xd), want_sm, dtype, f"softmax {dtype} 8x{cols}")
    _close(log_softmax(xd), ref.log_softmax(x), dtype, f"log_softmax {dtype} 8x{cols}")
    if dtype != torch.float32:
        _close(log_softmax(xd, -1, torch.float32), ref.log_softmax(x, -1, torch.float32),
               torch.float32, f"log_softmax {dtype}->fp32 8x{cols}")
    _close(logsumexp(xd), ref.logsumexp(x), dtype, f"logsumexp {dtype} 8x{cols}")


CE_ARGS = [dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0, HAS_SMOOTHING=False,
                SPLIT=False),
           dict(smoothing=0.0, logit_scale=0.5, lse_square_scale=0.0, HAS_SMOOTHING=False,
                SPLIT=False),
           dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0, HAS_SMOOTHING=False,
                SPLIT=True),
           # a scale whose products round (0.5 is exact): x * scale - m must
           # subtract the rounded product, not fuse into one FMA
           dict(smoothing=0.0, logit_scale=0.7, lse_square_scale=0.0, HAS_SMOOTHING=False,
                SPLIT=False)]


@pytest.mark.parametrize("cols", WIDTHS)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("ai", range(len(CE_ARGS)))
def test_cross_entropy_far_shifts(cols, dtype, ai):
    """Forward over one column block per row (the row kernel, the streaming
    kernel, or the split path for these few long rows) and over 1024-wide
    blocks; then the backward on the forward's lse."""
    p = CE_ARGS[ai]
    print(f"[gpu] far shifts cross entropy {dtype} 8x{cols} {p}", flush=True)
    x = _rows(dtype, cols, 7100 + cols)
    g = torch.Generator().manual_seed(7200 + cols)
    labels = torch.randint(0, cols, (8,), generator=g)
    labels[1] = cols // 3            # the spike row's label on its spike
    xd, ld = x.to(DEV), labels.to(DEV)
    for bs in sorted({max(1024, 1 << (cols - 1).bit_length()), 1024}):
        args = dict(ignored_index=-100, total_classes=cols, class_start_idx=0, BLOCK_SIZE=bs,
                    **p)
        got = cross_entropy_fwd(xd, ld, **args)
        want = ref.cross_entropy_fwd(x, labels, **args)
        n = 8 * -(-cols // bs)
        for k, (t, w) in enumerate(zip(got, want)):
            if k == 2 and p["SPLIT"]:
                continue
            _close(t.reshape(-1)[:n], w.reshape(-1)[:n], torch.float32,
                   f"ce fwd[{k}] {dtype} 8x{cols} bs {bs} {p}")
    if p["SPLIT"]:
        return
    lse = torch.logsumexp(x.float() * p["logit_scale"], dim=1)
    dloss = torch.rand(8, generator=g)
    bargs = (0.0, p["logit_scale"], 0.0, -100, cols, 0, 1 << 17, False)
    got = cross_entropy_bwd(dloss.to(DEV), xd, lse.to(DEV), ld, *bargs)
    want = ref.cross_entropy_bwd(dloss, x, lse, labels, *bargs)
    _close(got, want, dtype, f"ce bwd {dtype} 8x{cols} {p}")
