"""Pin the oracle (CPU tier).

The oracle (oracle/pytorch_impl.py) is the checker for every GPU parity test,
so it is itself checked here against things a plausible mistake cannot also
satisfy: an independent float64 numpy restatement, closed forms and
invariants, known answers, torch library routines the goldens reduce to in
special cases (F.cross_entropy with label smoothing / ignore_index, autograd
for the backward), brute-force per-program loops, and the committed golden
fixtures (tests/golden/, float64).
"""
import json
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ce_loops, numpy_ref
from oracle import pytorch_impl as ref

GOLDEN = __import__("pathlib").Path(__file__).parent / "golden"
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _close(a, b, atol, rtol):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    np.testing.assert_allclose(a, b, atol=atol, rtol=rtol, equal_nan=True)


# ---------------------------------------------------------------------------
# layer_norm
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(7, 33), (3, 5, 64), (16, 1024)])
def test_layer_norm_vs_numpy(shape):
    g = _g(1)
    x = torch.randn(shape, generator=g) * 3 + 1
    w = torch.randn(shape[-1], generator=g)
    b = torch.randn(shape[-1], generator=g)
    _close(ref.layer_norm(x, w, b), numpy_ref.layer_norm(x.numpy(), w.numpy(), b.numpy()),
           1e-5, 1e-5)


def test_layer_norm_invariants():
    g = _g(2)
    x = torch.randn(64, 256, generator=g) * 5 + 2
    y = ref.layer_norm(x, torch.ones(256), torch.zeros(256)).double()
    assert y.mean(dim=1).abs().max() < 1e-5
    var = x.double().var(dim=1, unbiased=False)
    # biased variance of the output is var / (var + eps); an unbiased variance fails this
    _close(y.var(dim=1, unbiased=False), var / (var + 1e-5), 1e-5, 1e-5)
    # all-equal rows normalize to 0, so the output is the bias
    b = torch.randn(256, generator=g)
    _close(ref.layer_norm(torch.full((4, 256), 3.25), torch.randn(256, generator=g), b),
           b.expand(4, 256), 1e-6, 0)


def test_layer_norm_eps_guard():
    x = torch.randn(2, 8)
    with pytest.raises(ValueError):
        ref.layer_norm(x, torch.ones(8), torch.zeros(8), eps=1e-6)


# ---------------------------------------------------------------------------
# rms_norm
# ---------------------------------------------------------------------------
def test_rms_norm_known_answer():
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0]])
    w = torch.tensor([1.0, 1.0, 2.0, 0.5])
    y = ref.rms_norm(x, (4,), w, eps=0.0)
    rms = math.sqrt((1 + 4 + 9 + 16) / 4)  # 2.7386...
    _close(y, [[1 / rms, 2 / rms, 6 / rms, 2 / rms]], 1e-6, 1e-6)


@pytest.mark.parametrize("shape,nshape", [((9, 40), (40,)), ((4, 6, 8), (6, 8))])
def test_rms_norm_vs_numpy(shape, nshape):
    g = _g(3)
    x = torch.randn(shape, generator=g)
    w = torch.randn(nshape, generator=g)
    _close(ref.rms_norm(x, nshape, w, 1e-5), numpy_ref.rms_norm(x.numpy(), nshape, w.numpy()),
           1e-5, 1e-5)


def test_rms_norm_scale_invariance_and_dtype():
    g = _g(4)
    x = torch.randn(8, 128, generator=g)
    w = torch.randn(128, generator=g)
    _close(ref.rms_norm(7.0 * x, (128,), w, 0.0), ref.rms_norm(x, (128,), w, 0.0), 1e-6, 1e-5)
    xb = x.to(torch.bfloat16)
    yb = ref.rms_norm(xb, (128,), w.to(torch.bfloat16), 1e-6)
    assert yb.dtype == torch.bfloat16


# ---------------------------------------------------------------------------
# softmax / log_softmax / logsumexp
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(4, 8), (100, 100), (2, 3, 4, 32), (128,)])
def test_softmax_family_vs_numpy(shape):
    x = 3 * torch.randn(shape, generator=_g(5))
    _close(ref.softmax(x), numpy_ref.softmax(x.numpy()), 1e-6, 1e-5)
    _close(ref.log_softmax(x), numpy_ref.log_softmax(x.numpy()), 1e-5, 1e-5)
    _close(ref.logsumexp(x), numpy_ref.logsumexp(x.numpy()), 1e-5, 1e-5)


def test_softmax_closed_forms():
    a, b = 0.3, -1.7
    p = ref.softmax(torch.tensor([a, b], dtype=torch.float64))
    _close(p[0], 1 / (1 + math.exp(b - a)), 1e-12, 1e-12)      # logistic
    x = torch.randn(16, 50, generator=_g(6), dtype=torch.float64)
    _close(ref.softmax(x).sum(-1), np.ones(16), 1e-12, 0)      # rows sum to one
    _close(ref.softmax(x + 11.5), ref.softmax(x), 1e-12, 1e-9)  # shift invariance
    _close(ref.softmax(torch.full((3, 40), 2.0)), np.full((3, 40), 1 / 40), 1e-7, 0)
    _close(ref.log_softmax(x), x - ref.logsumexp(x)[:, None], 1e-12, 1e-12)
    _close(ref.logsumexp(x + 4.25), ref.logsumexp(x) + 4.25, 1e-12, 1e-12)
    _close(ref.logsumexp(torch.full((2, 1000), -0.5, dtype=torch.float64)),
           np.full(2, -0.5 + math.log(1000)), 1e-12, 1e-12)


def test_log_softmax_dim_and_dtype():
    x = torch.randn(2, 8, 16, 8, generator=_g(7))
    _close(ref.log_softmax(x, dim=1), ref.log_softmax(x.transpose(1, 3), dim=-1).transpose(1, 3),
           1e-6, 1e-6)
    _close(ref.log_softmax(x, dim=1), numpy_ref.log_softmax(x.numpy(), axis=1), 1e-5, 1e-5)
    xh = x.to(torch.float16)
    assert ref.log_softmax(xh, dim=-1, dtype=torch.float32).dtype == torch.float32


def test_special_values_follow_torch():
    inf, nan = float("inf"), float("nan")
    x = torch.tensor([[0.0, 1.0, inf], [-inf, -inf, -inf], [0.0, nan, 1.0], [-inf, 0.0, 1.0]])
    lse = ref.logsumexp(x)
    assert lse[0] == inf and lse[1] == -inf and torch.isnan(lse[2])
    assert torch.isfinite(lse[3])
    sm = ref.softmax(x)
    assert torch.isnan(sm[0]).all() and torch.isnan(sm[1]).all() and torch.isnan(sm[2]).all()
    assert sm[3, 0] == 0 and torch.isfinite(sm[3]).all()
    _close(lse, numpy_ref.logsumexp(x.numpy()), 1e-6, 1e-6)


# ---------------------------------------------------------------------------
# cross entropy
# ---------------------------------------------------------------------------
REF_CE_CONFIGS = [  # ViperBench/cross_entropy/test.py:61-92
    dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1, total_classes=10,
         class_start_idx=0, BLOCK_SIZE=8, HAS_SMOOTHING=False, SPLIT=False),
    dict(smoothing=0.1, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1, total_classes=10,
         class_start_idx=0, BLOCK_SIZE=8, HAS_SMOOTHING=True, SPLIT=False),
    dict(smoothing=0.1, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1, total_classes=10,
         class_start_idx=0, BLOCK_SIZE=8, HAS_SMOOTHING=True, SPLIT=True),
    dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.1, ignored_index=-1, total_classes=10,
         class_start_idx=0, BLOCK_SIZE=4, HAS_SMOOTHING=False, SPLIT=False),
    dict(smoothing=0.0, logit_scale=0.5, lse_square_scale=0.05, ignored_index=-1, total_classes=10,
         class_start_idx=0, BLOCK_SIZE=4, HAS_SMOOTHING=False, SPLIT=False),
]
EXTRA_CE_CONFIGS = [
    dict(smoothing=0.2, logit_scale=1.3, lse_square_scale=0.01, ignored_index=3, total_classes=37,
         class_start_idx=0, BLOCK_SIZE=8, HAS_SMOOTHING=True, SPLIT=False),
    dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0, ignored_index=-100,
         total_classes=60, class_start_idx=10, BLOCK_SIZE=16, HAS_SMOOTHING=False, SPLIT=True),
    dict(smoothing=0.3, logit_scale=0.7, lse_square_scale=0.0, ignored_index=-100,
         total_classes=60, class_start_idx=-5, BLOCK_SIZE=4, HAS_SMOOTHING=True, SPLIT=True),
]


def _loops_flat(res, n):
    out = np.zeros(n)
    for k, v in res.items():
        out[k] = v
    return out


@pytest.mark.parametrize("cfg", REF_CE_CONFIGS + EXTRA_CE_CONFIGS)
@pytest.mark.parametrize("shape", [(4, 8), (5, 37)])
def test_ce_fwd_vs_loops(cfg, shape):
    g = _g(42)
    logits = torch.randn(shape, generator=g)
    labels = torch.randint(0, shape[1], (shape[0],), generator=g, dtype=torch.int32)
    labels[1] = cfg["ignored_index"]
    got = ref.cross_entropy_fwd(logits, labels, **cfg)
    want = ce_loops.cross_entropy_fwd(
        logits.double().tolist(), labels.tolist(), cfg["smoothing"], cfg["logit_scale"],
        cfg["lse_square_scale"], cfg["ignored_index"], cfg["total_classes"],
        cfg["class_start_idx"], cfg["BLOCK_SIZE"], cfg["HAS_SMOOTHING"], cfg["SPLIT"])
    n = shape[0] * shape[1]
    for t, w in zip(got, want):
        assert t.shape == shape and t.dtype == torch.float32
        _close(t.reshape(-1), _loops_flat(w, n), 2e-6, 2e-6)  # includes the zero tail


@pytest.mark.parametrize("smoothing", [0.0, 0.15])
def test_ce_one_block_equals_library(smoothing):
    g = _g(9)
    logits = 2 * torch.randn(32, 300, generator=g, dtype=torch.float64).float()
    labels = torch.randint(0, 300, (32,), generator=g)
    labels[::5] = -100
    loss, lse, z = ref.cross_entropy_fwd(logits, labels, smoothing, 1.0, 0.0, -100, 300, 0, 512,
                                         smoothing > 0, False)
    lib = F.cross_entropy(logits.double(), labels, reduction="none", ignore_index=-100,
                          label_smoothing=smoothing)
    _close(loss.reshape(-1)[:32], lib, 1e-5, 1e-5)
    _close(lse.reshape(-1)[:32], torch.logsumexp(logits.double(), dim=1), 1e-5, 1e-6)
    assert (z.reshape(-1)[:32] == 0).all()
    # mean over non-ignored rows equals the library's mean reduction
    keep = labels != -100
    _close(loss.reshape(-1)[:32][keep].double().mean(),
           F.cross_entropy(logits.double(), labels, ignore_index=-100, label_smoothing=smoothing),
           1e-6, 1e-6)


@pytest.mark.parametrize("smoothing", [0.0, 0.25])
def test_ce_split_is_vocab_parallel(smoothing):
    """SPLIT blocks are vocab shards: logsumexp over the block lse plus the sum
    of the SPLIT block losses is the full (label-smoothed) cross entropy."""
    g = _g(10)
    rows, cols, bs = 12, 96, 32
    logits = torch.randn(rows, cols, generator=g)
    labels = torch.randint(0, cols, (rows,), generator=g)
    loss, lse, _ = ref.cross_entropy_fwd(logits, labels, smoothing, 1.0, 0.0, -100, cols, 0, bs,
                                         smoothing > 0, True)
    nb = cols // bs
    blk_lse = lse.reshape(-1)[: nb * rows].view(nb, rows).double()
    blk_loss = loss.reshape(-1)[: nb * rows].view(nb, rows).double()
    full = torch.logsumexp(blk_lse, dim=0) + blk_loss.sum(dim=0)
    lib = F.cross_entropy(logits.double(), labels, reduction="none", label_smoothing=smoothing)
    _close(full, lib, 1e-5, 1e-5)


def test_ce_z_loss_and_shift():
    g = _g(11)
    logits = torch.randn(6, 40, generator=g)
    labels = torch.randint(0, 40, (6,), generator=g)
    l1, lse, z = ref.cross_entropy_fwd(logits, labels, 0.0, 1.0, 0.3, -100, 40, 0, 64, False, False)
    l0, _, _ = ref.cross_entropy_fwd(logits, labels, 0.0, 1.0, 0.0, -100, 40, 0, 64, False, False)
    _close((l1 - l0).reshape(-1)[:6], 0.3 * lse.reshape(-1)[:6].double() ** 2, 1e-5, 1e-5)
    _close(z.reshape(-1)[:6], 0.3 * lse.reshape(-1)[:6].double() ** 2, 1e-6, 1e-6)
    # class_start_idx shifts the label window: labels outside it give loss 0 (no smoothing)
    ls, _, _ = ref.cross_entropy_fwd(logits, labels + 100, 0.0, 1.0, 0.0, -100, 40, 100, 64,
                                     False, False)
    _close(ls, l0, 0, 0)
    lo, _, _ = ref.cross_entropy_fwd(logits, labels + 1000, 0.0, 1.0, 0.0, -100, 40, 100, 64,
                                     False, False)
    assert (lo == 0).all()


@pytest.mark.parametrize("smoothing,lss", [(0.0, 0.0), (0.0, 0.05), (0.2, 0.0)])
def test_ce_bwd_is_gradient(smoothing, lss):
    """One block, total_classes = n_cols: dlogits is the gradient of the forward
    loss (with z-loss term) scaled by dloss."""
    g = _g(12)
    rows, cols, scale = 8, 50, 0.8
    logits = torch.randn(rows, cols, generator=g, dtype=torch.float64)
    labels = torch.randint(0, cols, (rows,), generator=g)
    dloss = torch.rand(rows, generator=g, dtype=torch.float64)
    xl = logits.clone().requires_grad_(True)
    s = xl * scale
    lse = torch.logsumexp(s, dim=1)
    xy = s.gather(1, labels[:, None])[:, 0]
    loss = lse - smoothing * s.sum(1) / cols - (1 - smoothing) * xy + lss * lse * lse
    (loss * dloss).sum().backward()
    got = ref.cross_entropy_bwd(dloss.float(), logits.float(), lse.detach().float(), labels,
                                smoothing, scale, lss, -100, cols, 0, 64, smoothing > 0)
    _close(got, xl.grad, 2e-6, 1e-5)
    loops = ce_loops.cross_entropy_bwd(dloss.tolist(), logits.tolist(), lse.detach().tolist(),
                                       labels.tolist(), smoothing, scale, lss, -100, cols, 0,
                                       smoothing > 0)
    _close(got, loops, 2e-6, 1e-5)


def test_ce_bwd_ignored_rows_are_zero():
    logits = torch.randn(3, 16, generator=_g(13))
    labels = torch.tensor([2, -100, 5])
    lse = torch.logsumexp(logits, 1)
    d = ref.cross_entropy_bwd(torch.ones(3), logits, lse, labels, 0.0, 1.0, 0.0, -100, 16, 0, 8,
                              False)
    assert (d[1] == 0).all() and (d[0] != 0).any()


# ---------------------------------------------------------------------------
# golden fixtures (float64 expectations) vs the fp32 oracle
# ---------------------------------------------------------------------------
def _cases(npz):
    names = sorted({k.split("__")[0] for k in npz.files})
    return [(n, {k.split("__")[1]: npz[k] for k in npz.files if k.startswith(n + "__")})
            for n in names]


def _tol(dt):
    return {"f32": (2e-5, 2e-5), "f16": (2e-3, 2e-3), "bf16": (2e-2, 2e-2)}[dt]


def test_golden_fixtures_pin_oracle():
    for kernel in ("layer_norm", "rms_norm", "softmax", "log_softmax", "logsumexp"):
        with np.load(GOLDEN / f"{kernel}.npz") as npz:
            for name, c in _cases(npz):
                dt = str(c["dtype"])
                x = torch.from_numpy(c["x"]).to(DT[dt])
                if kernel == "layer_norm":
                    got = ref.layer_norm(x, torch.from_numpy(c["w"]).to(DT[dt]),
                                         torch.from_numpy(c["b"]).to(DT[dt]))
                elif kernel == "rms_norm":
                    got = ref.rms_norm(x, (x.shape[-1],), torch.from_numpy(c["w"]).to(DT[dt]),
                                       float(c["eps"]))
                elif kernel == "log_softmax":
                    got = ref.log_softmax(x, dim=int(c.get("dim", -1)))
                else:
                    got = getattr(ref, kernel)(x)
                atol, rtol = _tol(dt)
                try:
                    _close(got.float(), c["expected"], atol, rtol)
                except AssertionError as e:
                    raise AssertionError(f"{kernel}/{name}: {e}") from None
    with np.load(GOLDEN / "cross_entropy.npz") as npz:
        for name, c in _cases(npz):
            p = json.loads(str(c["params"]))
            got = ref.cross_entropy_fwd(torch.from_numpy(c["logits"]),
                                        torch.from_numpy(c["labels"]), **p)
            rows = c["logits"].shape[0]
            ncb = -(-c["logits"].shape[1] // p["BLOCK_SIZE"])
            n = rows * ncb
            for t, key in zip(got, ("loss", "lse", "z_loss")):
                _close(t.reshape(-1)[:n], c[key][:n], 2e-5, 2e-5)


# ---------------------------------------------------------------------------
# sibling reductions: mean / max / argmax
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dim,keep", [((64, 128), 0, False), ((64, 128), 1, True),
                                            ((2, 3, 4, 5), [1, 2], False), ((8, 16, 32), 2, False),
                                            ((3, 4, 5), [0, 2], True)])
def test_mean_reduction_vs_numpy(shape, dim, keep):
    x = torch.randn(shape, generator=_g(20))
    _close(ref.mean_reduction(x, dim, keep), numpy_ref.mean(x.numpy(), dim, keep), 1e-6, 1e-5)
    # dtype casts first: a bf16 input with dtype=float32 equals the mean of its fp32 values
    xb = x.to(torch.bfloat16)
    _close(ref.mean_reduction(xb, dim, keep, torch.float32),
           numpy_ref.mean(xb.float().numpy(), dim, keep), 1e-6, 1e-5)


def test_max_argmax_semantics():
    nan, inf = float("nan"), float("inf")
    x = torch.tensor([[1., 3., 3., 2.], [1., nan, 5., nan], [-inf] * 4, [2., inf, inf, 0.]])
    v, i = ref.max_reduction(x, 1)
    # first maximal position; NaN is the largest value; an all -inf row gives index 0
    assert i.tolist() == [1, 1, 0, 1]
    assert v[0] == 3 and torch.isnan(v[1]) and v[2] == -inf and v[3] == inf
    assert ref.argmax(x, 1).tolist() == [1, 1, 0, 1]
    nv, ni = numpy_ref.max_argmax(x.numpy(), 1)
    assert ni.tolist() == [1, 1, 0, 1]
    g = torch.randn(16, 33, 7, generator=_g(21))
    for d in (0, 1, 2):
        rv, ri = ref.max_reduction(g, d, keepdim=True)
        nv, ni = numpy_ref.max_argmax(g.numpy(), d, keepdims=True)
        _close(rv, nv, 0, 0)
        assert (ri.numpy() == ni).all()
        assert (ref.argmax(g, d).numpy() == np.squeeze(ni, d)).all()
    with pytest.raises(TypeError):
        ref.max_reduction([1, 2], 0)
