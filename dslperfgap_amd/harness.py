"""Measurement harness for the HIP backend on one MI355X.

MI355X counterparts of the reference's timing and roofline helpers:

* ``profile_fn``     wall-clock median with a synchronize on both sides of every
                     call, 10 warm-up + 100 timed calls (ViperBench/benchmark.py:26-58);
* ``time_kernel``    per-call device-event timing, median/mean/min
                     (experiments/_harness.py:110-139);
* ``essential_work`` algorithmic bytes of one call -- the norm/softmax rule of
                     experiments/exp_cliff_roofline.py:229-234 (read x + write y),
                     plus the logsumexp and cross-entropy models the reference lacks;
* ``PEAKS`` / ``select_peak``  an MI355X entry (vendor HBM figure) next to the
                     measured stream-copy rate (exp_cliff_roofline.py:192-218);
* ``Rotation``       HBM-resident copies of a workload's inputs and outputs that
                     successive launches cycle through, so that no launch finds its
                     data in the 256 MB Infinity Cache (MALL) or the L2;
* ``copy_peak``      the sustained device-to-device copy rate (vbh_stream_copy),
                     the yardstick of kernels that read and write about as much;
* ``read_peak``      the sustained streaming-read rate (vbh_stream_read), the
                     yardstick of kernels that write almost nothing (logsumexp,
                     the cross-entropy forward, mean / max / argmax).

The timed launches go straight through the C ABI with preallocated buffers
(what ``hip_impl`` calls after its checks and allocation), so host overhead per
launch is a few microseconds and the GPU is kept busy.
"""
from __future__ import annotations

import math
import statistics
import time
from dataclasses import dataclass
from typing import Callable

import torch

from . import _bridge, _lib
from .workloads import Workload

# vendor figures for context; the measured stream-copy rate is the bar
PEAKS = {
    "MI355X": dict(memory=8.0e12, note="AMD Instinct MI355X: 288 GB HBM3E, 8.0 TB/s (vendor)"),
    "MI300X": dict(memory=5.3e12, note="AMD Instinct MI300X: 192 GB HBM3, 5.3 TB/s (vendor)"),
}


def select_peak(device_name: str):
    """(bytes/s, note) of the vendor HBM figure for a device name, or (None, reason)."""
    up = device_name.upper()
    for key, tbl in PEAKS.items():
        if key in up:
            return tbl["memory"], tbl["note"]
    if "GFX950" in up or "MI355" in up or "MI350" in up:
        return PEAKS["MI355X"]["memory"], PEAKS["MI355X"]["note"]
    return None, f"no peak-table entry for '{device_name}'"


# kernels that write almost nothing: quoted against the measured streaming-read
# rate; every other kernel reads and writes about as much and is quoted against
# the measured copy rate
READ_DOMINATED = frozenset({"logsumexp", "cross_entropy", "argmax", "max_reduction",
                            "mean_reduction"})


def peak_kind(kernel: str) -> str:
    """"read" or "copy": the measured yardstick of a kernel."""
    return "read" if kernel in READ_DOMINATED else "copy"


def essential_work(kernel: str, inputs) -> int:
    """Algorithmic HBM bytes of one call: every input read once, every output written once."""
    el = lambda t: t.element_size() * t.numel()  # noqa: E731
    x = inputs[0]
    if kernel in ("softmax", "log_softmax"):
        return 2 * el(x)
    if kernel == "layer_norm":
        w, b = inputs[1], inputs[2]
        return 2 * el(x) + el(w) + (el(b) if b is not None else 0)
    if kernel == "rms_norm":
        return 2 * el(x) + el(inputs[2])
    if kernel == "logsumexp":
        n = x.shape[-1] if x.dim() else 1
        return el(x) + (x.numel() // max(n, 1)) * x.element_size()
    if kernel == "cross_entropy_bwd":
        # dloss, logits, lse, labels -> dlogits (same shape and dtype as logits)
        dloss, logits, lse, labels = inputs[:4]
        rows = logits.shape[0]
        return 2 * el(logits) + el(labels) + rows * lse.element_size() + rows * dloss.element_size()
    if kernel == "cross_entropy":
        logits, labels, bs = inputs[0], inputs[1], int(inputs[8])
        rows, cols = logits.shape
        return el(logits) + el(labels) + 3 * 4 * rows * math.ceil(cols / bs)
    if kernel in ("argmax", "max_reduction", "mean_reduction"):
        # read x once; outputs: int64 indices and/or one value per reduced slice
        dim = inputs[1]
        n = x.shape[dim] if isinstance(dim, int) else math.prod(x.shape[d] for d in dim)
        outs = x.numel() // max(n, 1)
        per_out = {"argmax": 8, "max_reduction": 8 + x.element_size(),
                   "mean_reduction": x.element_size()}[kernel]
        return el(x) + outs * per_out
    raise KeyError(kernel)


def library_fn(kernel: str):
    """torch's own GPU implementation of a kernel: the library row that E_lib
    (t_library / t_backend, experiments/_harness.py:142-146) is measured against.
    layer_norm / softmax / log_softmax / logsumexp are the ATen calls the goldens
    make; rms_norm is the golden's eager formula (rms_norm/pytorch_impl.py:8-10);
    cross_entropy is torch's fused F.cross_entropy (per-row losses), the library
    form of the same computation for one column block."""
    import torch.nn.functional as F

    if kernel == "layer_norm":
        return lambda x, w, b, eps=1e-5: F.layer_norm(x, tuple(w.shape), w, b, eps)
    if kernel == "rms_norm":
        def rms(x, normalized_shape, w, eps=1e-5):
            dims = tuple(range(x.ndim - len(normalized_shape), x.ndim))
            r = torch.sqrt(torch.mean(x.float() ** 2, dim=dims, keepdim=True) + eps)
            return ((x.float() / r) * w.float()).to(x.dtype)
        return rms
    if kernel == "softmax":
        return lambda x: F.softmax(x, dim=-1)
    if kernel == "log_softmax":
        return lambda x, dim=-1, dtype=None: F.log_softmax(x, dim=dim, dtype=dtype)
    if kernel == "logsumexp":
        return lambda x: torch.logsumexp(x, dim=-1)
    if kernel == "cross_entropy":
        return lambda logits, labels, *a: F.cross_entropy(logits, labels, reduction="none")
    if kernel == "argmax":
        return lambda x, dim, keepdim=False: torch.argmax(x, dim=dim, keepdim=keepdim)
    if kernel == "max_reduction":
        return lambda x, dim, keepdim=False: torch.max(x, dim, keepdim=keepdim)
    if kernel == "mean_reduction":
        return lambda x, dim, keepdim=False, dtype=None: torch.mean(x, dim, keepdim=keepdim,
                                                                    dtype=dtype)
    raise KeyError(kernel)


def profile_fn(fn, args, warmup: int = 10, iters: int = 100) -> float:
    """Median wall-clock ms of fn(*args), synchronizing around every call."""
    for _ in range(warmup):
        fn(*args)
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn(*args)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    times.sort()
    return times[len(times) // 2]


def time_kernel(launch: Callable[[int], None], reps: int = 50, warmup: int = 15,
                before: Callable[[int], None] | None = None) -> dict:
    """Per-launch device-event timing on the current stream (ms)."""
    for i in range(warmup):
        if before:
            before(i)
        launch(i)
    torch.cuda.synchronize()
    times = []
    for i in range(reps):
        if before:
            before(i)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        launch(i)
        e.record()
        e.synchronize()
        times.append(s.elapsed_time(e))
    times.sort()
    return {"median_ms": times[len(times) // 2], "mean_ms": statistics.fmean(times),
            "min_ms": times[0], "reps": reps}


def time_back_to_back(launch: Callable[[int], None], steps: int, warmup: int,
                      fence=None) -> dict:
    """`steps` launches back to back, bracketed by synchronize and device events.

    `fence`, if given, is a context manager entered after the warm-up launches
    have completed and left once the timed launches have (a profiler range that
    holds exactly the timed dispatches).  Returns the event time and the wall
    time of the whole timed region (ms)."""
    import contextlib

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with fence if fence is not None else contextlib.nullcontext():
        t0 = time.perf_counter()
        s.record()
        for i in range(steps):
            launch(warmup + i)
        e.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
    return {"event_ms": s.elapsed_time(e), "wall_ms": wall, "steps": steps}


def warm_gpu(launch: Callable[[int], None], seconds: float = 0.5) -> int:
    """Run `launch` back to back for about `seconds` so that clocks and page
    tables are at steady state before a timed region; returns launches made."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(16):
            launch(n)
            n += 1
        torch.cuda.synchronize()
    return n


def copy_peak(device, nbytes: int = 4 << 30, reps: int = 20) -> float:
    """Sustained device-to-device copy rate in bytes/s (read + write counted)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=device)
    src.fill_(1)
    stream = _bridge.stream(torch.device(device))

    def launch(_):
        _lib.call("vbh_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, stream)

    warm_gpu(launch, 0.3)
    r = time_back_to_back(launch, reps, 3)
    del src, dst
    return 2.0 * nbytes * reps / (r["event_ms"] * 1e-3)


def read_peak(device, nbytes: int = 4 << 30, reps: int = 20) -> float:
    """Sustained streaming-read rate in bytes/s (bytes read; the one 32-bit
    word written per workgroup is not counted)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    src.fill_(1)
    pbytes = _lib.lib().vbh_stream_read_partial_bytes(nbytes)
    partial = torch.empty(pbytes, dtype=torch.uint8, device=device)
    stream = _bridge.stream(torch.device(device))

    def launch(_):
        _lib.call("vbh_stream_read", src.data_ptr(), nbytes, partial.data_ptr(), pbytes, stream)

    warm_gpu(launch, 0.3)
    r = time_back_to_back(launch, reps, 3)
    del src, partial
    return 1.0 * nbytes * reps / (r["event_ms"] * 1e-3)


def copy_rotation(device, traffic_bytes: int, min_footprint: int = 2 << 30):
    """(launch, bytes moved per launch, copies): stream copies that each move
    `traffic_bytes` (half read, half written, rounded down to 16-byte vectors),
    cycling through enough buffers that no launch hits the Infinity Cache."""
    half = max(16, (traffic_bytes // 2) // 16 * 16)
    copies = max(2, math.ceil(min_footprint / (2 * half)))
    bufs = [(torch.empty(half, dtype=torch.uint8, device=device),
             torch.empty(half, dtype=torch.uint8, device=device)) for _ in range(copies)]
    for a, _ in bufs:
        a.fill_(1)
    stream = _bridge.stream(torch.device(device))

    def launch(k):
        a, b = bufs[k % copies]
        _lib.call("vbh_stream_copy", a.data_ptr(), b.data_ptr(), half, stream)

    launch.buffers = bufs  # keep the buffers alive as long as the launcher
    return launch, 2 * half, copies


def read_rotation(device, nbytes: int, min_footprint: int = 2 << 30):
    """(launch, bytes read per launch, copies): streaming reads of `nbytes`
    (rounded down to 16-byte vectors) cycling through enough buffers that no
    launch hits the Infinity Cache -- the read-only counterpart of
    copy_rotation, the yardstick at a read-only kernel's own size."""
    size = max(16, nbytes // 16 * 16)
    copies = max(2, math.ceil(min_footprint / size))
    bufs = [torch.empty(size, dtype=torch.uint8, device=device) for _ in range(copies)]
    for a in bufs:
        a.fill_(1)
    pbytes = _lib.lib().vbh_stream_read_partial_bytes(size)
    partial = torch.empty(pbytes, dtype=torch.uint8, device=device)
    stream = _bridge.stream(torch.device(device))

    def launch(k):
        _lib.call("vbh_stream_read", bufs[k % copies].data_ptr(), size, partial.data_ptr(),
                  pbytes, stream)

    launch.buffers = (bufs, partial)  # kept alive as long as the launcher
    return launch, size, copies


def runtime_copy_rotation(device, traffic_bytes: int, min_footprint: int = 2 << 30):
    """(launch, bytes moved per launch, copies): the HIP runtime's own
    device-to-device copy (torch's ``copy_`` between contiguous buffers of one
    GPU, a hipMemcpyAsync) of ``traffic_bytes / 2`` bytes per launch, cycling
    through enough buffer pairs that no launch hits the Infinity Cache -- a
    same-size yardstick that is not this library's own code."""
    half = max(16, (traffic_bytes // 2) // 16 * 16)
    copies = max(2, math.ceil(min_footprint / (2 * half)))
    bufs = [(torch.empty(half, dtype=torch.uint8, device=device),
             torch.empty(half, dtype=torch.uint8, device=device)) for _ in range(copies)]
    for a, _ in bufs:
        a.fill_(1)

    def launch(k):
        a, b = bufs[k % copies]
        b.copy_(a)

    launch.buffers = bufs
    return launch, 2 * half, copies


def capture_graph(launch: Callable[..., None], launches: int):
    """A HIP graph (torch.cuda.CUDAGraph) holding `launches` consecutive
    launches, launch(k, stream) for k = 0 .. launches - 1 on the capture
    stream, after one eager pass of them on a side stream; replayed 3 times."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        for k in range(launches):
            launch(k, torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = torch.cuda.current_stream().cuda_stream
        for k in range(launches):
            launch(k, st)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    return graph


def graph_replay_ms(launch: Callable[..., None], launches: int, replays: int = 20) -> dict:
    """Device time per launch when `launches` consecutive launches (launch(k,
    stream) for k = 0 .. launches - 1) are captured into one HIP graph and the
    graph is replayed `replays` times back to back: the launch sequence with no
    host work between kernels.  Returns the per-launch ms (events around the
    replays) and the launch count."""
    graph = capture_graph(launch, launches)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        graph.replay()
    e.record()
    e.synchronize()
    ms = s.elapsed_time(e) / (replays * launches)
    del graph
    return {"ms_per_launch": ms, "launches_per_graph": launches, "replays": replays}


def ce_mean_step(rot: "Rotation", n_rows: int):
    """(launch, scalars): the cross-entropy forward of a rotation's copy k
    followed by the scalar mean of its first n_rows losses on the GPU
    (vbh_reduce_fwd, mean over the contiguous loss.view(-1)[:n_rows]) -- the
    full step of a mean-reduced loss.  scalars[k % copies] holds copy k's mean."""
    dev = rot.outputs[0][0].device
    scalars = [torch.empty((), dtype=torch.float32, device=dev) for _ in range(rot.copies)]
    losses = [o[0].data_ptr() for o in rot.outputs]
    outs = [t.data_ptr() for t in scalars]
    stream = _bridge.stream(dev)
    call = _lib.call
    copies = rot.copies

    def launch(k, st=stream):
        rot.launch(k, st)
        call("vbh_reduce_fwd", losses[k % copies], outs[k % copies], None, 1, n_rows, 1,
             _lib.F32, _lib.F32, _lib.REDUCE_MEAN, st)

    return launch, scalars


def copy_rate_at(device, traffic_bytes: int, reps: int = 200,
                 min_footprint: int = 2 << 30) -> float:
    """Copy rate (bytes/s, read + write) when one launch moves `traffic_bytes`
    (half read, half written), cycling through enough buffers that no launch
    hits the Infinity Cache: the achievable rate at a kernel's own size."""
    launch, moved, copies = copy_rotation(device, traffic_bytes, min_footprint)
    warm_gpu(launch, 0.3)
    r = time_back_to_back(launch, reps, 2 * copies)
    del launch
    return 1.0 * moved * reps / (r["event_ms"] * 1e-3)


@dataclass
class Rotation:
    """Device copies of a workload and a launcher that cycles through them."""

    workload: Workload
    copies: int
    launch: Callable[[int], None]
    outputs: list
    inputs: list


def _float_code(t):
    return _bridge.FLOAT_CODES[t.dtype]


def make_rotation(w: Workload, cpu_args: tuple, device, min_footprint: int = 2 << 30) -> Rotation:
    """Place ceil(min_footprint / bytes_per_launch) (at least 2) copies of the
    workload's tensors in HBM and return a launcher for copy i % copies."""
    copies = max(2, math.ceil(min_footprint / w.bytes_per_launch))
    dev = torch.device(device)
    stream = _bridge.stream(dev)
    ins, outs = [], []
    x0 = cpu_args[1] if w.fn == "cross_entropy_bwd" else cpu_args[0]
    for _ in range(copies):
        ins.append(tuple(a.to(dev) if isinstance(a, torch.Tensor) else a for a in cpu_args))
    p = _bridge.ptr
    if w.fn in ("layer_norm", "rms_norm", "softmax", "log_softmax"):
        for _ in range(copies):
            outs.append(torch.empty(x0.shape, dtype=x0.dtype, device=dev))
    elif w.fn == "logsumexp":
        for _ in range(copies):
            outs.append(torch.empty(x0.shape[:-1], dtype=x0.dtype, device=dev))
    elif w.fn == "cross_entropy_fwd":
        for _ in range(copies):
            outs.append(tuple(torch.empty(x0.shape, dtype=torch.float32, device=dev)
                              for _ in range(3)))
    elif w.fn == "cross_entropy_bwd":
        for _ in range(copies):
            outs.append(torch.empty(x0.shape, dtype=x0.dtype, device=dev))
    rows = x0.numel() // x0.shape[-1]
    cols = x0.shape[-1]
    dt = _float_code(x0)
    call = _lib.call

    if w.fn == "layer_norm":
        eps = float(cpu_args[3])
        wdt = _float_code(cpu_args[1])
        argv = [(p(i[0]), p(i[1]), p(i[2]), p(o)) for i, o in zip(ins, outs)]

        def launch(k, st=stream):
            a = argv[k % copies]
            call("vbh_layer_norm_fwd", a[0], a[1], a[2], a[3], rows, cols, eps, dt, wdt, st)
    elif w.fn == "rms_norm":
        eps = float(cpu_args[3])
        wdt = _float_code(cpu_args[2])
        argv = [(p(i[0]), p(i[2]), p(o)) for i, o in zip(ins, outs)]

        def launch(k, st=stream):
            a = argv[k % copies]
            call("vbh_rms_norm_fwd", a[0], a[1], a[2], rows, cols, eps, dt, wdt, st)
    elif w.fn in ("softmax", "log_softmax"):
        mode = 1 if w.fn == "log_softmax" else 0
        argv = [(p(i[0]), p(o)) for i, o in zip(ins, outs)]

        def launch(k, st=stream):
            a = argv[k % copies]
            call("vbh_softmax_fwd", a[0], a[1], rows, cols, dt, dt, mode, st)
    elif w.fn == "logsumexp":
        argv = [(p(i[0]), p(o)) for i, o in zip(ins, outs)]

        def launch(k, st=stream):
            a = argv[k % copies]
            call("vbh_logsumexp_fwd", a[0], a[1], rows, cols, dt, dt, st)
    elif w.fn == "cross_entropy_fwd":
        (_, labels, sm, scale, lss, ign, total, start, bs, has_sm, split) = cpu_args
        ldt = _bridge.LABEL_CODES[labels.dtype]
        argv = [(p(i[0]), p(i[1]), p(o[0]), p(o[1]), p(o[2])) for i, o in zip(ins, outs)]

        def launch(k, st=stream):
            a = argv[k % copies]
            call("vbh_cross_entropy_fwd", a[0], a[1], dt, ldt, a[2], a[3], a[4], rows, cols, cols,
                 float(sm), float(scale), float(lss), int(ign), int(total), int(start), int(bs),
                 int(has_sm), int(split), st)
    elif w.fn == "cross_entropy_bwd":
        (_, _, _, labels, sm, scale, lss, ign, total, start, _bs, has_sm) = cpu_args
        ldt = _bridge.LABEL_CODES[labels.dtype]
        argv = [(p(i[0]), p(i[1]), p(i[2]), p(i[3]), p(o)) for i, o in zip(ins, outs)]

        def launch(k, st=stream):
            a = argv[k % copies]
            call("vbh_cross_entropy_bwd", a[0], a[1], a[2], a[3], a[4], dt, ldt, rows, cols, cols,
                 cols, 1, float(sm), float(scale), float(lss), int(ign), int(total), int(start),
                 int(has_sm), st)
    else:
        raise KeyError(w.fn)
    return Rotation(w, copies, launch, outs, ins)
