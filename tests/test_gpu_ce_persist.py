"""GPU parity of the persistent cross-entropy forward (ce_fwd_persist).

Launches of at least 1024 fp32 rows of one column block and at least two
32 KiB chunks (16384 columns) take the persistent kernel by default: one
workgroup per CU folding its rows chunk by chunk into per-lane online (max,
sum of exp) pairs, in workgroups of 256 lanes from 64 chunks per CU up and of
512 below; the tune flag TUNE_PERSIST takes it down to one chunk (8192
columns) and any row count, and with a block override of 256 or 512 sets the
workgroup size (both are run on every case here).  16-bit logits and column
blocks stay on
ce_fwd_rows (cases below as well).  These tests hold it to the oracle (the restated
golden, oracle/pytorch_impl.py) at the strict fp32 tolerance of the measured
configs, on every output, with the golden's special values (NaN, +inf, all
-inf rows, -inf chunks inside finite rows, rows at +-FLT_MAX), shifted labels,
ignored rows, int32 / int64 labels, smoothing, z-loss, SPLIT and negative
logit scales; and, forced by the tune flags, on launches of a few segments
(workgroups with one, two or no segments, odd chunk counts) and against
ce_fwd_rows on the same inputs.
"""
import pytest
import torch

from dslperfgap_amd import _lib
from dslperfgap_amd.viperbench.cross_entropy.hip_impl import cross_entropy_fwd
from oracle import pytorch_impl as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

PARAMS = [
    dict(smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0, HAS_SMOOTHING=False, SPLIT=False),
    dict(smoothing=0.1, logit_scale=0.7, lse_square_scale=1e-4, HAS_SMOOTHING=True, SPLIT=False),
    dict(smoothing=0.0, logit_scale=1.3, lse_square_scale=1e-4, HAS_SMOOTHING=False, SPLIT=True),
    dict(smoothing=0.2, logit_scale=-0.5, lse_square_scale=0.0, HAS_SMOOTHING=True, SPLIT=False),
]


def _g(seed):
    return torch.Generator().manual_seed(seed)


def setup_module(module):
    print(f"[gpu] device: {torch.cuda.get_device_name(0)}", flush=True)
    _lib.lib()


def _check(got, want, n, what, split=False):
    """allclose on the n valid block-major positions of each output (fp32
    outputs whatever the logits' dtype), NaN positions matching; z_loss is not
    compared under SPLIT (cross_entropy/test.py:28-58)."""
    for k, (t, w) in enumerate(zip(got, want)):
        if k == 2 and split:
            continue
        g = t.reshape(-1)[:n].float().cpu()
        e = w.reshape(-1)[:n].float().cpu()
        ok = torch.allclose(g, e, atol=1e-5, rtol=1e-5, equal_nan=True)
        if not ok:
            bad = ~torch.isclose(g, e, atol=1e-5, rtol=1e-5, equal_nan=True)
            idx = bad.nonzero().flatten()[:8].tolist()
            raise AssertionError(f"{what} output {k}: {int(bad.sum())} mismatches, first at "
                                 + ", ".join(f"{i} (got {g[i].item()}, want {e[i].item()})"
                                             for i in idx))


# (flags, block) of vbh_tune_override for the persistent kernel's launches:
# the default choice, then each workgroup size forced
SHAPES = [(0, 0), (_lib.TUNE_PERSIST, 256), (_lib.TUNE_PERSIST, 512)]


def _run_shapes(fn, what):
    """fn() under each of SHAPES; returns the outputs' valid rows per shape."""
    outs = []
    try:
        for flags, block in SHAPES:
            _lib.tune_override(_lib.OP_CROSS_ENTROPY, 0, block, flags)
            print(f"[ce persist] {what} flags={flags} block={block}", flush=True)
            outs.append(fn(f"{what} flags={flags} block={block}"))
    finally:
        _lib.tune_override(_lib.OP_CROSS_ENTROPY, 0, 0, 0)
    return outs


def _inputs(rows, cols, dtype, seed, start, specials=True):
    g = _g(seed)
    logits = 2 * torch.randn(rows, cols, generator=g)
    labels = torch.randint(0, cols + start, (rows,), generator=g)
    labels[5::11] = -100
    if specials and rows >= 12:
        big = torch.finfo(torch.float32).max
        logits[0, : cols // 2] = float("-inf")   # whole -inf chunks, finite row
        labels[0] = start + cols - 3
        logits[1, :] = float("-inf")              # all -inf: NaN lse
        logits[2, cols // 3] = float("inf")       # +inf: NaN
        logits[3, 11] = float("nan")              # NaN
        logits[4, :] = -big if dtype == torch.float32 else -3.0e38   # all at -FLT_MAX
        logits[6, 7] = 3.0e38                     # one huge finite logit
        labels[6] = start + 7
        # rows whose loss would cancel terms of 1e30 or 1e6 (the fp32 rounding
        # of the sum of logits is not the oracle's): their lse only
        logits[7, 100:] = -1e30                   # a far shift in later chunks
        labels[7] = -100
        logits[8, -1] = 50.0                      # the row max in the last vector
        labels[8] = start + cols - 1
        logits[9, :] = 1e6                        # large equal logits
        labels[9] = -100
        logits[10, :1000] = float("-inf")         # label on a -inf logit
        labels[10] = start + 3
    return logits.to(dtype), labels


@pytest.mark.parametrize("rows,cols,bs,dtype", [
    (1024, 16384, 16384, torch.float32),   # two full chunks
    (1024, 24576, 24576, torch.float32),   # three full chunks
    (1030, 24580, 24580, torch.float32),   # four chunks, the last of one vector
    (1100, 32000, 32000, torch.float32),   # C4's row: four chunks, the last of 1856 vectors
    (1024, 8200, 8200, torch.bfloat16),    # ce_fwd_rows: 16-bit logits
    (600, 16384, 8192, torch.float32),     # ce_fwd_rows: two column blocks per row
])
@pytest.mark.parametrize("pi", range(len(PARAMS)))
@pytest.mark.parametrize("ldt", [torch.int64, torch.int32])
def test_persistent_cross_entropy_matches_oracle(rows, cols, bs, dtype, pi, ldt):
    p = PARAMS[pi]
    start = cols // 7
    logits, labels = _inputs(rows, cols, dtype, 700 + rows + pi, start)
    labels = labels.to(ldt)
    args = dict(ignored_index=-100, total_classes=cols + start, class_start_idx=start,
                BLOCK_SIZE=bs, **p)
    want = ref.cross_entropy_fwd(logits, labels, **args)
    n = rows * (cols // bs)
    xd, ld = logits.to(DEV), labels.to(DEV)

    def run(what):
        got = cross_entropy_fwd(xd, ld, **args)
        _check(got, want, n, what, p["SPLIT"])

    tag = f"{rows}x{cols} bs={bs} {dtype} {ldt} params {pi}"
    if dtype == torch.float32 and bs == cols:
        _run_shapes(run, tag)
    else:
        print(f"[ce persist] {tag}", flush=True)
        run(tag)


@pytest.mark.parametrize("rows", [1, 3, 12, 257, 300])
@pytest.mark.parametrize("cols,dtype", [(8192, torch.float32), (8200, torch.float32),
                                        (12292, torch.float32), (20000, torch.float32)])
def test_persistent_cross_entropy_forced_few_segments(rows, cols, dtype):
    """Forced persistent launches of fewer segments than CUs or a few per
    workgroup; and the forced row kernel on the same inputs."""
    start = 3
    logits, labels = _inputs(rows, cols, dtype, 800 + rows, start)
    p = PARAMS[1]
    args = dict(ignored_index=-100, total_classes=cols + start, class_start_idx=start,
                BLOCK_SIZE=cols, **p)
    want = ref.cross_entropy_fwd(logits, labels, **args)
    outs = []
    try:
        for flags, block in ((_lib.TUNE_PERSIST, 256), (_lib.TUNE_PERSIST, 512),
                             (_lib.TUNE_NO_PERSIST, 0)):
            _lib.tune_override(_lib.OP_CROSS_ENTROPY, 0, block, flags)
            what = f"rows={rows} cols={cols} {dtype} flags={flags} block={block}"
            print(f"[ce persist] forced {what}", flush=True)
            got = cross_entropy_fwd(logits.to(DEV), labels.to(DEV), **args)
            _check(got, want, rows, what)
            outs.append([t.reshape(-1)[:rows].cpu() for t in got])
    finally:
        _lib.tune_override(_lib.OP_CROSS_ENTROPY, 0, 0, 0)
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.allclose(a, b, atol=1e-5, rtol=1e-5, equal_nan=True), \
                (a - b).abs().max()


def test_persistent_cross_entropy_repeatable():
    """Two launches on the same inputs give bit-identical outputs (each
    segment's fold order is fixed by the grid, not by timing), for the
    default and each forced workgroup size."""
    rows, cols = 2048, 24576
    logits, labels = _inputs(rows, cols, torch.float32, 900, 0, specials=False)
    xd, ld = logits.to(DEV), labels.to(DEV)
    args = (0.1, 1.0, 1e-4, -100, cols, 0, cols, True, False)

    def run(what):
        a = [t.clone() for t in cross_entropy_fwd(xd, ld, *args)]
        b = cross_entropy_fwd(xd, ld, *args)
        for x, y in zip(a, b):
            assert torch.equal(x.reshape(-1)[:rows], y.reshape(-1)[:rows]), what

    _run_shapes(run, f"repeat {rows}x{cols}")


@pytest.mark.parametrize("rows,cols,pad", [(1030, 16388, 4), (300, 8192, 12)])
def test_persistent_cross_entropy_strided_rows(rows, cols, pad):
    """Rows `pad` elements apart beyond their width (a column slice of a wider
    buffer): the persistent kernel reads each row from its own stride; 300
    rows forced with TUNE_PERSIST (256 lanes), 1030 by default."""
    g = _g(950 + rows)
    big = 2 * torch.randn(rows, cols + pad, generator=g)
    logits = big[:, :cols]
    labels = torch.randint(0, cols, (rows,), generator=g)
    labels[7] = -100
    args = (0.1, 1.0, 1e-4, -100, cols, 0, cols, True, False)
    bd = big.to(DEV)
    print(f"[ce persist] strided {rows}x{cols} pad {pad}", flush=True)
    try:
        if rows < 1024:
            _lib.tune_override(_lib.OP_CROSS_ENTROPY, 0, 256, _lib.TUNE_PERSIST)
        got = cross_entropy_fwd(bd[:, :cols], labels.to(DEV), *args)
    finally:
        _lib.tune_override(_lib.OP_CROSS_ENTROPY, 0, 0, 0)
    want = ref.cross_entropy_fwd(logits, labels, *args)
    _check(got, want, rows, f"strided {rows}x{cols} pad {pad}")
