"""vbh_cross_entropy_fwd_noalloc against vbh_cross_entropy_fwd_ws (GPU).

The no-allocation entry point runs the same kernels as the workspace entry
point, with the split's segment results in the library's static per-GPU
scratch instead of a caller workspace, so its outputs must be bit-identical.
Two calls in a row on shapes that take the row split (the second smaller,
so it reads the scratch the first one left behind only where it wrote it
itself), then one that does not split; both entry points are called through
the C ABI.
"""
import pytest
import torch

from dslperfgap_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _case(rows, cols, seed, smoothing=0.0, ignore_some=False):
    g = torch.Generator().manual_seed(seed)
    logits = (2.0 * torch.randn(rows, cols, generator=g)).to(DEV)
    labels = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int64)
    if ignore_some:
        labels[::3] = -100
    return logits, labels.to(DEV), smoothing


def _run(name, logits, labels, smoothing, ws=None):
    rows, cols = logits.shape
    outs = [torch.full((rows, cols), float("nan"), device=DEV) for _ in range(3)]
    stream = torch.cuda.current_stream().cuda_stream
    args = [logits.data_ptr(), labels.data_ptr(), _lib.F32, _lib.I64,
            *(o.data_ptr() for o in outs), rows, cols, cols, float(smoothing), 1.0, 0.1, -100,
            cols, 0, cols, int(smoothing > 0), 0]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    _lib.call(name, *args, stream)
    return outs


@pytest.mark.parametrize("order", ["big_then_small"])
def test_noalloc_matches_the_workspace_entry_point(order):
    print(f"[gpu] no-alloc cross entropy: {order}", flush=True)
    cases = [(64, 128256, 1, 0.0, False), (8, 65536, 2, 0.1, True), (512, 4096, 3, 0.0, False)]
    for rows, cols, seed, sm, ign in cases:
        need = _lib.cross_entropy_workspace_bytes(rows, cols, cols, _lib.F32)
        if (rows, cols) != (512, 4096):
            assert 0 < need <= 32 << 10, (rows, cols, need)
        else:
            assert need == 0
        logits, labels, sm = _case(rows, cols, seed, sm, ign)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
        want = _run("vbh_cross_entropy_fwd_ws", logits, labels, sm, ws)
        got = _run("vbh_cross_entropy_fwd_noalloc", logits, labels, sm)
        torch.cuda.synchronize()
        n = rows  # one column block per row: positions [0, rows) of each output
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a.reshape(-1)[:n], b.reshape(-1)[:n]), (rows, cols, i)
            assert bool(torch.isfinite(a.reshape(-1)[:n]).all()), (rows, cols, i)
