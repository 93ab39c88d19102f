"""ViperBench-style latency profile of the HIP backend on one MI355X.

The counterpart of ViperBench/benchmark.py:26-58, 350-450 for this family: for
each of the reference benchmark's own cases (small and large per kernel,
``workloads.REFERENCE_CASES``) and the five measured configs, it times

* ``hip``      the drop-in ``hip_impl`` function, and
* ``pytorch``  torch's own GPU implementation (``harness.library_fn``),

with the reference's protocol -- ``profile_fn``: wall-clock median of
single calls with a synchronize on both sides, 10 warm-up + 100 calls (3 + 5
for the cases the reference marks slow), and peak ``max_memory_allocated`` of
one call -- and adds device-side columns the reference lacks: the median
device-event time of one launch on inputs that cycle through >= 2 GiB of HBM
(no Infinity Cache hits), the achieved GB/s over the algorithmic bytes, and
E_lib = t_pytorch / t_hip x 100 (experiments/_harness.py:142-146) on device
times.  Rows are written in the reference's profile.csv column order, extra
columns appended.

    python -m dslperfgap_amd.viperbench.benchmark [--out profile.MI355X.csv]
"""
from __future__ import annotations

import argparse
import csv
import importlib
import math
import sys

import torch

from dslperfgap_amd import harness
from dslperfgap_amd.workloads import REFERENCE_CASES, WORKLOADS, to_device

FIELDS = ["kernel", "size", "impl", "input_desc", "latency_ms", "peak_memory_mb",
          "device_us", "achieved_GBps", "e_lib_pct"]


def _hip_fn(kernel: str, fn: str):
    mod = importlib.import_module(f"dslperfgap_amd.viperbench.{kernel}.hip_impl")
    return getattr(mod, fn)


def profile_fn_mem(fn, args, warmup, iters):
    """The reference's profile_fn: (median wall ms, peak MB of one call)."""
    lat = harness.profile_fn(fn, args, warmup=warmup, iters=iters)
    torch.cuda.reset_peak_memory_stats()
    torch.cuda.synchronize()
    fn(*args)
    torch.cuda.synchronize()
    return lat, torch.cuda.max_memory_allocated() / (1024 * 1024)


def device_time_us(fn, cpu_args, traffic_bytes, reps=50, min_footprint=2 << 30):
    """Median device-event time of one call, inputs cycling through HBM copies."""
    copies = max(2, math.ceil(min_footprint / max(traffic_bytes, 1)))
    copies = min(copies, 64)
    sets = [to_device(cpu_args, "cuda") for _ in range(copies)]
    harness.warm_gpu(lambda k: fn(*sets[k % copies]), 0.3)
    r = harness.time_kernel(lambda k: fn(*sets[k % copies]), reps=reps, warmup=2 * copies)
    del sets
    torch.cuda.empty_cache()
    return r["median_ms"] * 1e3


def cases(include_configs=True):
    out = [(c.kernel, c.size, c.fn, c.desc, c.make, c.is_slow) for c in REFERENCE_CASES]
    if include_configs:
        for w in WORKLOADS.values():
            if w.fn == "cross_entropy_bwd":
                continue  # the reference's benchmark has no backward rows
            out.append((w.kernel, w.key, w.fn, w.desc, w.make, w.fn == "cross_entropy_fwd"))
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default="profile.MI355X.csv")
    ap.add_argument("--kernels", nargs="*", default=None)
    ap.add_argument("--no-configs", action="store_true", help="reference cases only")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    rows = []
    print(f"{'Kernel':<14} {'Size':<17} {'Impl':<8} {'Latency(ms)':>11} {'PeakMem(MB)':>11} "
          f"{'device_us':>10} {'GB/s':>8} {'E_lib%':>8}  Input", flush=True)
    for kernel, size, fn_name, desc, make, is_slow in cases(not args.no_configs):
        if args.kernels and kernel not in args.kernels:
            continue
        warmup, iters = (3, 5) if is_slow else (10, 100)
        cpu_args = make()
        dev_args = to_device(cpu_args, "cuda")
        traffic = harness.essential_work(kernel, dev_args)
        impls = [("pytorch", harness.library_fn(kernel)), ("hip", _hip_fn(kernel, fn_name))]
        dev_us = {}
        for impl, fn in impls:
            torch.cuda.empty_cache()
            lat, mem = profile_fn_mem(fn, dev_args, warmup, iters)
            dev_us[impl] = device_time_us(fn, cpu_args, traffic)
            gbps = traffic / (dev_us[impl] * 1e-6) / 1e9
            e_lib = 100.0 * dev_us["pytorch"] / dev_us[impl]
            rows.append({"kernel": kernel, "size": size, "impl": impl, "input_desc": desc,
                         "latency_ms": round(lat, 4), "peak_memory_mb": round(mem, 2),
                         "device_us": round(dev_us[impl], 2), "achieved_GBps": round(gbps, 1),
                         "e_lib_pct": round(e_lib, 1)})
            print(f"{kernel:<14} {size:<17} {impl:<8} {lat:>11.4f} {mem:>11.2f} "
                  f"{dev_us[impl]:>10.2f} {gbps:>8.1f} {e_lib:>8.1f}  {desc}", flush=True)
        del dev_args
    with open(args.out, "w", newline="") as f:
        writer = csv.DictWriter(f, fieldnames=FIELDS)
        writer.writeheader()
        writer.writerows(rows)
    print(f"\nResults written to {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
