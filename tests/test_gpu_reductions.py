"""GPU parity of the sibling row reductions (mean / max / argmax).

The HIP path is compared with the oracle (oracle/pytorch_impl.py) on the same
seeded inputs: means with allclose at the reference's loose fp32 tolerance
(ViperBench/test_utils.py:12-25, x2), max values and all indices exactly
(ViperBench/argmax/test.py:38-42 compares indices with torch.equal).
"""
import pytest
import torch

from dslperfgap_amd import _lib
from dslperfgap_amd.viperbench.argmax.hip_impl import argmax
from dslperfgap_amd.viperbench.max_reduction.hip_impl import max_reduction
from dslperfgap_amd.viperbench.mean_reduction.hip_impl import mean_reduction
from oracle import pytorch_impl as ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = {torch.float32: 2e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _same(got, want, what=""):
    assert got.device.type == "cuda", what
    assert got.shape == want.shape and got.dtype == want.dtype, (what, got.shape, want.shape,
                                                                 got.dtype, want.dtype)
    g, w = got.cpu(), want
    if g.is_floating_point():
        ok = torch.equal(g.isnan(), w.isnan()) and torch.equal(g[~g.isnan()], w[~w.isnan()])
    else:
        ok = torch.equal(g, w)
    assert ok, f"{what}: results differ"


def _close(got, want, what=""):
    assert got.shape == want.shape and got.dtype == want.dtype, (what, got.shape, want.shape)
    tol = TOL[want.dtype]
    assert torch.allclose(got.float().cpu(), want.float(), atol=tol, rtol=tol, equal_nan=True), what


MEAN_CASES = [((64, 128), 0, False), ((64, 128), 1, True), ((2, 3, 4, 5), [1, 2], False),
              ((8, 16, 32), 2, False)]  # mean_reduction/test.py:12-33
MAX_CASES = [((128, 256), 0, False), ((256, 128), 1, False), ((32, 64, 128), 2, False),
             ((64, 256), 1, True), ((16, 32, 64), -1, False)]  # max_reduction/test.py:13-38
ARGMAX_CASES = [((128, 256), 0, False), ((256, 128), 1, False), ((32, 64, 128), 2, False),
                ((16, 32, 64), 1, True)]  # argmax/test.py:13-33


@pytest.mark.parametrize("shape,dim,keep", MEAN_CASES)
def test_mean_reference_cases(shape, dim, keep):
    x = torch.randn(shape, generator=_g(300))
    _close(mean_reduction(x.to(DEV), dim, keep), ref.mean_reduction(x, dim, keep))


@pytest.mark.parametrize("shape,dim,keep", MAX_CASES)
def test_max_reference_cases(shape, dim, keep):
    x = torch.randn(shape, generator=_g(301))
    v, i = max_reduction(x.to(DEV), dim, keep)
    rv, ri = ref.max_reduction(x, dim, keep)
    _same(v, rv, "values")
    _same(i, ri, "indices")


@pytest.mark.parametrize("shape,dim,keep", ARGMAX_CASES)
def test_argmax_reference_cases(shape, dim, keep):
    x = torch.randn(shape, generator=_g(302))
    _same(argmax(x.to(DEV), dim, keep), ref.argmax(x, dim, keep))


@pytest.mark.parametrize("shape,dtype", [((1024, 1024), torch.float16), ((8192, 32768), torch.float16),
                                         ((1024, 1024), torch.float32),
                                         ((8192, 32768), torch.float32)])
def test_benchmark_shapes(shape, dtype):
    """ViperBench/benchmark.py:274-291 (and argmax :89-97): dim = 1."""
    print(f"[gpu] reductions {shape} {dtype}", flush=True)
    x = torch.randn(shape, generator=_g(303)).to(dtype)
    xd = x.to(DEV)
    v, i = max_reduction(xd, 1)
    rv, ri = ref.max_reduction(x, 1)
    _same(v, rv, "max values")
    _same(i, ri, "max indices")
    _same(argmax(xd, 1), ref.argmax(x, 1), "argmax")
    if dtype == torch.float32:
        _close(mean_reduction(xd, 1), ref.mean_reduction(x, 1), "mean")


@pytest.mark.parametrize("cols_per_vec", [12, 16, 17, 32, 33, 64, 65, 96])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_max_argmax_both_lane_loops(cols_per_vec, dtype):
    """Row lengths around the switch between the two max / argmax lane loops
    (the search after the loop where every lane holds a batch of vectors or
    more, the per-vector search below): the row's maximum tied across vectors,
    in the first or last vector of a lane, NaN first or last, and all -inf
    rows; values and indices exactly."""
    vn = 16 // torch.empty(0, dtype=dtype).element_size()
    cols = cols_per_vec * vn
    g = _g(900 + cols)
    rows = 48
    x = torch.randint(-5, 6, (rows, cols), generator=g).float()
    for r in range(rows):
        k = r % 6
        if k == 0:
            x[r, 0] = 9.0
            x[r, cols - 1] = 9.0         # tie between the first and the last element
        elif k == 1:
            x[r, cols - vn] = 9.0       # first element of the last vector
        elif k == 2:
            x[r, vn - 1] = 9.0          # last element of the first vector
            x[r, cols // 2] = 9.0
        elif k == 3:
            x[r, cols - 1] = float("nan")
        elif k == 4:
            x[r, 1] = float("nan")
            x[r, cols - 2] = float("nan")
        else:
            x[r, :] = float("-inf")
    x = x.to(dtype)
    xd = x.to(DEV)
    v, i = max_reduction(xd, 1)
    rv, ri = ref.max_reduction(x, 1)
    _same(v, rv, f"values cols={cols}")
    _same(i, ri, f"indices cols={cols}")
    _same(argmax(xd, 1), ref.argmax(x, 1), f"argmax cols={cols}")


@pytest.mark.parametrize("cols", [1, 7, 64, 100, 1000, 4096, 65537])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_widths_ties_and_special_values(cols, dtype):
    g = _g(304)
    x = torch.randint(-3, 4, (40, cols), generator=g).float()  # many ties
    x[1, cols // 2] = float("nan")
    x[2, :] = float("-inf")
    x[3, cols - 1] = float("inf")
    x[4, cols // 3] = float("nan")
    x[4, cols - 1] = float("nan")
    x = x.to(dtype)
    xd = x.to(DEV)
    v, i = max_reduction(xd, 1)
    rv, ri = ref.max_reduction(x, 1)
    _same(v, rv, f"values cols={cols}")
    _same(i, ri, f"indices cols={cols}")
    _same(argmax(xd, -1), ref.argmax(x, -1), f"argmax cols={cols}")
    y = torch.randn(40, cols, generator=g).to(dtype)
    _close(mean_reduction(y.to(DEV), 1), ref.mean_reduction(y, 1), f"mean cols={cols}")
    _close(mean_reduction(y.to(DEV), 0, True), ref.mean_reduction(y, 0, True), "mean dim0")


def test_dims_dtype_and_degenerate():
    g = _g(305)
    x = torch.randn(3, 4, 5, 6, generator=g)
    xd = x.to(DEV)
    for dims in ([0, 2], [1, 3], [0, 1, 2, 3], [3, 1], -1, None):
        _close(mean_reduction(xd, dims, True), ref.mean_reduction(x, dims, True), f"dims={dims}")
    xb = x.to(torch.bfloat16)
    _close(mean_reduction(xb.to(DEV), [1, 2], False, torch.float32),
           ref.mean_reduction(xb, [1, 2], False, torch.float32), "bf16 -> fp32")
    _close(mean_reduction(xd, 1, False, torch.float16),
           ref.mean_reduction(x, 1, False, torch.float16), "fp32 -> fp16 cast first")
    e = torch.empty(4, 0)
    _close(mean_reduction(e.to(DEV), 1), ref.mean_reduction(e, 1), "empty axis -> NaN")
    z = torch.empty(0, 5)  # empty outer axis: empty results, no error
    _same(argmax(z.to(DEV), 1), ref.argmax(z, 1), "empty outer argmax")
    _same(argmax(z.to(DEV), 1, True), ref.argmax(z, 1, True), "empty outer argmax keepdim")
    v, i = max_reduction(z.to(DEV), 1, True)
    rv, ri = ref.max_reduction(z, 1, True)
    _same(v, rv, "empty outer max values")
    _same(i, ri, "empty outer max indices")
    _close(mean_reduction(z.to(DEV), 1), ref.mean_reduction(z, 1), "empty outer mean")
    s = torch.tensor(1.5)
    _same(argmax(s.to(DEV), 0), ref.argmax(s, 0), "0-d argmax")
    _same(argmax(x.to(DEV), None), ref.argmax(x, None), "flattened argmax")
    v, i = max_reduction(s.to(DEV), 0)
    rv, ri = ref.max_reduction(s, 0)
    _same(v, rv)
    _same(i, ri)
    base = torch.randn(40 * 1000 + 1, generator=g)
    (bd,) = (base.to(DEV),)
    _same(argmax(bd[1:].view(40, 1000), 1), ref.argmax(base[1:].view(40, 1000), 1), "unaligned")


@pytest.mark.parametrize("tpr,block", [(1, 64), (16, 256), (64, 64), (192, 384), (1024, 1024)])
def test_reduce_geometry_overrides(tpr, block):
    x = torch.randn(33, 3001, generator=_g(306))
    xd = x.to(DEV)
    try:
        _lib.tune_override(_lib.OP_REDUCE, tpr, block, 0)
        v, i = max_reduction(xd, 1)
        rv, ri = ref.max_reduction(x, 1)
        _same(v, rv)
        _same(i, ri)
        _close(mean_reduction(xd, 1), ref.mean_reduction(x, 1))
    finally:
        _lib.tune_override(_lib.OP_REDUCE, 0, 0, 0)


# ---------------------------------------------------------------------------
# few long rows: the split path (segments reduced in parallel, then combined)
# ---------------------------------------------------------------------------
SPLIT_SHAPES = [(1, 131072), (3, 131072), (17, 262144), (200, 131072)]


@pytest.mark.parametrize("rows,cols", SPLIT_SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_split_reductions_match_the_oracle(rows, cols, dtype):
    """These launches split every row (the workspace query says so); special
    values sit in different segments: the row maximum twice (ties across
    segments give the first), and, in other rows, a NaN after an earlier
    maximum or two NaNs (the first NaN wins)."""
    code = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[dtype]
    for op in (_lib.REDUCE_MEAN, _lib.REDUCE_MAX, _lib.REDUCE_ARGMAX):
        assert _lib.reduce_workspace_bytes(rows, cols, 1, code, op) > 0, (rows, cols, op)
    x = torch.randn(rows, cols, generator=_g(310 + rows)).to(dtype)
    x[0, cols // 3] = 50.0
    x[0, cols - 5] = 50.0
    if rows > 1:
        x[1, 7] = 60.0
        x[1, cols // 2 + 1] = float("nan")
    if rows > 2:
        x[2, cols - 1] = float("nan")
        x[2, cols // 4] = float("nan")
        x[2, 3] = float("inf")
    xd = x.to(DEV)
    what = f"{rows}x{cols} {dtype}"
    v, i = max_reduction(xd, 1)
    rv, ri = ref.max_reduction(x, 1)
    _same(v, rv, "max values " + what)
    _same(i, ri, "max indices " + what)
    _same(argmax(xd, 1), ref.argmax(x, 1), "argmax " + what)
    _same(argmax(xd, -1, True), ref.argmax(x, -1, True), "argmax keepdim " + what)
    xm = torch.randn(rows, cols, generator=_g(320 + rows)).to(dtype) + 3.0
    xmd = xm.to(DEV)
    _close(mean_reduction(xmd, 1), ref.mean_reduction(xm, 1), "mean " + what)
    if dtype != torch.float32:
        _close(mean_reduction(xmd, 1, False, torch.float32),
               ref.mean_reduction(xm, 1, False, torch.float32), "mean fp32 out " + what)


def test_split_reduction_falls_back_without_enough_workspace():
    """vbh_reduce_fwd_ws with a workspace smaller than the query's size (or
    none) runs the unsplit kernel: the same indices and values."""
    rows, cols = 5, 65536
    x = torch.randn(rows, cols, generator=_g(330)).to(DEV)
    need = _lib.reduce_workspace_bytes(rows, cols, 1, _lib.F32, _lib.REDUCE_MAX)
    assert need > 0
    outs = []
    for ws_bytes in (need, need - 16, 0):
        v = torch.empty(rows, device=DEV)
        i = torch.empty(rows, dtype=torch.int64, device=DEV)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=DEV)
        _lib.call("vbh_reduce_fwd_ws", x.data_ptr(), v.data_ptr(), i.data_ptr(), rows, cols, 1,
                  _lib.F32, _lib.F32, _lib.REDUCE_MAX, ws.data_ptr() if ws_bytes else None,
                  ws_bytes, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append((v.cpu(), i.cpu()))
    for v, i in outs[1:]:
        assert torch.equal(v, outs[0][0]) and torch.equal(i, outs[0][1])
    rv, ri = ref.max_reduction(x.cpu(), 1)
    assert torch.equal(outs[0][1], ri)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_misaligned_rows_reductions(dtype):
    """Rows not a multiple of the 16-byte vector (head / aligned body / tail):
    every residue of n modulo the vector width; the maximum in a head, in a
    tail and tied between the two, a NaN in a head or a tail; max, argmax
    exactly, mean at tolerance."""
    vn = 16 // torch.empty(0, dtype=dtype).element_size()
    for n in [4 * vn + r for r in range(1, vn)] + [50257]:
        rows = 2 * vn + 3
        x = torch.randn(rows, n, generator=_g(700 + n)).to(dtype)
        for r in range(rows):
            if r % 4 == 0:
                x[r, 0] = 40.0                 # head of this row (or first body element)
            elif r % 4 == 1:
                x[r, n - 1] = 40.0             # tail
            elif r % 4 == 2:
                x[r, 1] = 40.0
                x[r, n - 2] = 40.0             # tie: the first wins
        x[3, 0] = float("nan")
        x[7, n - 1] = float("nan")
        x[7, n // 2] = 41.0
        xd = x.to(DEV)
        what = f"misaligned {dtype} n={n}"
        v, i = max_reduction(xd, 1)
        rv, ri = ref.max_reduction(x, 1)
        _same(v, rv, "max values " + what)
        _same(i, ri, "max indices " + what)
        _same(argmax(xd, 1), ref.argmax(x, 1), "argmax " + what)
        xm = torch.randn(rows, n, generator=_g(710 + n)).to(dtype) + 2.0
        _close(mean_reduction(xm.to(DEV), 1), ref.mean_reduction(xm, 1), "mean " + what)
