"""A battery of calls that reaches every kernel of libvbhip at least once:
each row kernel (register-resident, persistent guarded and unguarded,
streaming, rows that are not whole vectors), the split first and second
stages, the middle-axis kernels, the cross-entropy forward / combine /
backward, the no-allocation entry point and the copy / read yardsticks.

``run()`` returns {case name: output tensor on the CPU}.  The debug-bounds
test runs it once under the release library (in the pytest process) and once
under the bounds-checked debug library (``python tests/_bounds_battery.py OUT``
with VBHIP_LIB naming libvbhip_debug.so), then compares the outputs and reads
the debug library's count of failed checks.  Inputs are seeded on the CPU, so
both runs see the same values.
"""
import os
import sys

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

import torch  # noqa: E402

from dslperfgap_amd import _lib  # noqa: E402
from dslperfgap_amd.viperbench.argmax.hip_impl import argmax  # noqa: E402
from dslperfgap_amd.viperbench.cross_entropy.hip_impl import (  # noqa: E402
    cross_entropy_bwd, cross_entropy_fwd)
from dslperfgap_amd.viperbench.layer_norm.hip_impl import layer_norm  # noqa: E402
from dslperfgap_amd.viperbench.log_softmax.hip_impl import log_softmax  # noqa: E402
from dslperfgap_amd.viperbench.logsumexp.hip_impl import logsumexp  # noqa: E402
from dslperfgap_amd.viperbench.max_reduction.hip_impl import max_reduction  # noqa: E402
from dslperfgap_amd.viperbench.mean_reduction.hip_impl import mean_reduction  # noqa: E402
from dslperfgap_amd.viperbench.rms_norm.hip_impl import rms_norm  # noqa: E402
from dslperfgap_amd.viperbench.softmax.hip_impl import softmax  # noqa: E402

DEV = "cuda:0"


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _x(rows, cols, seed, dtype=torch.float32, scale=1.0):
    return (scale * torch.randn(rows, cols, generator=_g(seed))).to(dtype).to(DEV)


def _override(op, flags, block=0):
    class _Ctx:
        def __enter__(self):
            _lib.tune_override(op, 0, block, flags)

        def __exit__(self, *exc):
            _lib.tune_override(op, 0, 0, 0)
    return _Ctx()


def run() -> dict:
    out = {}
    # LayerNorm / RMSNorm: one row group per workgroup, persistent (guarded fp32,
    # unguarded bf16), rows not whole vectors, rows beyond the register budget
    for dt, cols in ((torch.float32, 1024), (torch.bfloat16, 4096), (torch.bfloat16, 20480)):
        x = _x(96, cols, 1, dt)
        w = (1 + 0.1 * torch.randn(cols, generator=_g(2))).to(dt).to(DEV)
        b = (0.1 * torch.randn(cols, generator=_g(3))).to(dt).to(DEV)
        for name, flags in (("rows", _lib.TUNE_NO_PERSIST), ("pipe", _lib.TUNE_PERSIST)):
            with _override(_lib.OP_LAYER_NORM, flags):
                out[f"ln {dt} {cols} {name}"] = layer_norm(x, w, b)
            with _override(_lib.OP_RMS_NORM, flags):
                out[f"rms {dt} {cols} {name}"] = rms_norm(x, (cols,), w, 1e-6)
    for cols in (1001, 70000):  # not whole vectors; wider than the register budget
        x = _x(9, cols, 4)
        w = (1 + 0.1 * torch.randn(cols, generator=_g(5))).to(DEV)
        b = (0.1 * torch.randn(cols, generator=_g(6))).to(DEV)
        out[f"ln {cols}"] = layer_norm(x, w, b)
        out[f"ln {cols} no bias"] = layer_norm(x, w, None)
        out[f"rms {cols}"] = rms_norm(x, (cols,), w)
    # softmax family: rows, rows not whole vectors, split rows (both stages),
    # split rows not whole vectors, streaming rows, a middle axis
    for rows, cols, dt in ((64, 4096, torch.float32), (33, 1001, torch.float32),
                           (40, 2048, torch.float16), (7, 131072, torch.float32),
                           (5, 131075, torch.float32), (130, 70000, torch.float32)):
        x = _x(rows, cols, 7, dt, 3.0)
        key = f"{rows}x{cols} {dt}"
        out[f"softmax {key}"] = softmax(x)
        out[f"log_softmax {key}"] = log_softmax(x)
        out[f"logsumexp {key}"] = logsumexp(x)
    x3 = (3 * torch.randn(6, 40, 24, generator=_g(8))).to(DEV)
    out["log_softmax dim 1"] = log_softmax(x3, 1)
    out["log_softmax dim 0 fp32 out"] = log_softmax(x3.half(), 0, torch.float32)
    out["logsumexp 600x70000"] = logsumexp(_x(600, 70000, 9, scale=2.0))
    # cross entropy forward: column blocks, labels int32 / int64, rows not whole
    # vectors, split rows (segments + combine), streaming segments; backward tiles
    for rows, cols, bs, ldt in ((64, 1000, 256, torch.int64), (33, 1001, 1024, torch.int32),
                                (7, 131072, 131072, torch.int64),
                                (5, 131075, 131075, torch.int32),
                                (600, 70000, 131072, torch.int64)):
        logits = _x(rows, cols, 10, scale=2.0)
        labels = torch.randint(0, cols, (rows,), generator=_g(11)).to(ldt)
        labels[1] = -100
        for sm in (0.0, 0.1):
            res = cross_entropy_fwd(logits, labels.to(DEV), sm, 0.9, 0.01, -100, cols, 0, bs,
                                    sm > 0, False)
            # the valid block-major positions only: the rest of each [rows, cols]
            # output is left unwritten (as in the reference's Triton backend), so
            # it holds whatever the allocator's block held before
            n = rows * -(-cols // bs)
            for i, t in enumerate(res):
                out[f"ce {rows}x{cols} bs{bs} sm{sm} out{i}"] = t.reshape(-1)[:n].clone()
    # the persistent forward (forced: a few rows, the last chunk of a row partly
    # past its end, int32 labels, smoothing; workgroups of 256 and 512 lanes)
    rows, cols = 40, 20000
    logits = _x(rows, cols, 17, scale=2.0)
    labels = torch.randint(0, cols, (rows,), generator=_g(18)).to(torch.int32)
    labels[3] = -100
    for lanes in (256, 512):
        with _override(_lib.OP_CROSS_ENTROPY, _lib.TUNE_PERSIST, lanes):
            res = cross_entropy_fwd(logits, labels.to(DEV), 0.1, 0.9, 0.01, -100, cols, 0, cols,
                                    True, False)
        for i, t in enumerate(res):
            out[f"ce persistent {rows}x{cols} {lanes} lanes out{i}"] = t.reshape(-1)[:rows].clone()
    for rows, cols, dt in ((48, 3000, torch.float32), (37, 1001, torch.float32),
                           (37, 4099, torch.bfloat16)):
        logits = _x(rows, cols, 12, dt)
        labels = torch.randint(0, cols, (rows,), generator=_g(13))
        labels[5] = -100
        dloss = torch.rand(rows, generator=_g(14)).to(DEV)
        lse = torch.logsumexp(logits.float() * 0.9, dim=1)
        out[f"ce bwd {rows}x{cols} {dt}"] = cross_entropy_bwd(
            dloss, logits, lse, labels.to(DEV), 0.05, 0.9, 0.02, -100, cols, 0, 8192, True)
    # the no-allocation forward (split rows: the static scratch)
    rows, cols = 8, 65536
    logits = _x(rows, cols, 15, scale=2.0)
    labels = torch.randint(0, cols, (rows,), generator=_g(16)).to(DEV)
    res = [torch.zeros(rows, cols, device=DEV) for _ in range(3)]
    _lib.call("vbh_cross_entropy_fwd_noalloc", logits.data_ptr(), labels.data_ptr(), _lib.F32,
              _lib.I64, *(t.data_ptr() for t in res), rows, cols, cols, 0.0, 1.0, 0.0, -100,
              cols, 0, cols, 0, 0, torch.cuda.current_stream().cuda_stream)
    for i, t in enumerate(res):
        out[f"ce noalloc out{i}"] = t
    # mean / max / argmax: rows, rows not whole vectors, split rows, a middle axis
    for rows, cols, dt in ((64, 1000, torch.float16), (33, 1001, torch.float32),
                           (3, 131072, torch.float32)):
        x = _x(rows, cols, 17, dt)
        key = f"{rows}x{cols} {dt}"
        out[f"mean {key}"] = mean_reduction(x, 1)
        v, i = max_reduction(x, 1)
        out[f"max {key}"], out[f"max idx {key}"] = v, i
        out[f"argmax {key}"] = argmax(x, 1)
        out[f"mean dim0 {key}"] = mean_reduction(x, 0)
        out[f"argmax dim0 {key}"] = argmax(x, 0)
    # the yardsticks
    nbytes = 1 << 20
    src = torch.randint(0, 1 << 30, (nbytes // 4,), generator=_g(18), dtype=torch.int32).to(DEV)
    dst = torch.zeros_like(src)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.call("vbh_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, stream)
    out["stream copy"] = dst
    pbytes = _lib.lib().vbh_stream_read_partial_bytes(nbytes)
    partial = torch.zeros(pbytes // 4, dtype=torch.int32, device=DEV)
    _lib.call("vbh_stream_read", src.data_ptr(), nbytes, partial.data_ptr(), pbytes, stream)
    out["stream read"] = partial
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in out.items()}


def slack_probe() -> dict:
    """With 16 bytes of slack the last 16-byte vector of every buffer fails its
    check: a softmax of one [4, 256] fp32 tensor then skips that vector's load
    and store.  Returns the count and place of the failed checks and whether
    the skipped output bytes kept their sentinel."""
    _lib.debug_bounds(clear=True)
    x = _x(4, 256, 19)
    y = torch.full_like(x, 7.0)
    _lib.debug_bounds_slack(16)
    try:
        _lib.call("vbh_softmax_fwd", x.data_ptr(), y.data_ptr(), 4, 256, _lib.F32, _lib.F32, 0,
                  torch.cuda.current_stream().cuda_stream)
        failed, where = _lib.debug_bounds(clear=True)
    finally:
        _lib.debug_bounds_slack(0)
    yc = y.cpu()
    return {"failed": failed, "where": where,
            "tail_untouched": bool((yc.reshape(-1)[-4:] == 7.0).all()),
            "rest_written": bool((yc.reshape(-1)[:-4] != 7.0).all())}


if __name__ == "__main__":
    # child process: VBHIP_LIB names the debug library
    _lib.lib()
    _lib.debug_bounds(clear=True)
    outs = run()
    failed, where = _lib.debug_bounds(clear=True)
    probe = slack_probe()
    after_failed, _ = _lib.debug_bounds(clear=True)
    torch.save({"outs": outs, "failed": failed, "where": where, "probe": probe,
                "after_failed": after_failed}, sys.argv[1])
    print(f"[bounds] {len(outs)} outputs, {failed} failed checks, probe {probe}", flush=True)
