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

A case or an implementation that raises does not end the sweep: as in
ViperBench/benchmark.py:388-428, it gets a row whose measured columns read
``ERROR`` (the message is printed), and the next one runs; the CSV is written
at the end either way.

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


def measure(fn, dev_args, cpu_args, traffic, warmup, iters) -> dict:
    """One implementation on one case: the reference protocol's latency and
    peak memory, and the HBM-cycled device time."""
    torch.cuda.empty_cache()
    lat, mem = profile_fn_mem(fn, dev_args, warmup, iters)
    return {"latency_ms": lat, "peak_memory_mb": mem,
            "device_us": device_time_us(fn, cpu_args, traffic)}


def impls_for(kernel: str, fn_name: str):
    return [("pytorch", lambda: harness.library_fn(kernel)),
            ("hip", lambda: _hip_fn(kernel, fn_name))]


def _error_row(kernel, size, impl, desc, err) -> dict:
    msg = f"{type(err).__name__}: {err}"[:80]
    print(f"{kernel:<14} {size:<17} {impl:<8} {'ERROR':>11}  {msg}", flush=True)
    return {"kernel": kernel, "size": size, "impl": impl, "input_desc": desc,
            "latency_ms": "ERROR", "peak_memory_mb": "ERROR", "device_us": "ERROR",
            "achieved_GBps": "ERROR", "e_lib_pct": ""}


def run_cases(case_list, impls=impls_for, measure_fn=measure, to_dev=to_device) -> list[dict]:
    """Profile every (case, implementation); a failure gives an ERROR row and
    the sweep goes on."""
    rows = []
    for kernel, size, fn_name, desc, make, is_slow in case_list:
        warmup, iters = (3, 5) if is_slow else (10, 100)
        try:
            cpu_args = make()
            dev_args = to_dev(cpu_args, "cuda")
            traffic = harness.essential_work(kernel, dev_args)
        except Exception as e:  # inputs could not be built: every impl errs
            rows += [_error_row(kernel, size, impl, desc, e) for impl, _ in
                     impls(kernel, fn_name)]
            continue
        dev_us = {}
        for impl, get_fn in impls(kernel, fn_name):
            try:
                m = measure_fn(get_fn(), dev_args, cpu_args, traffic, warmup, iters)
            except Exception as e:
                rows.append(_error_row(kernel, size, impl, desc, e))
                continue
            dev_us[impl] = m["device_us"]
            gbps = traffic / (m["device_us"] * 1e-6) / 1e9
            e_lib = (100.0 * dev_us["pytorch"] / m["device_us"]) if "pytorch" in dev_us else None
            rows.append({"kernel": kernel, "size": size, "impl": impl, "input_desc": desc,
                         "latency_ms": round(m["latency_ms"], 4),
                         "peak_memory_mb": round(m["peak_memory_mb"], 2),
                         "device_us": round(m["device_us"], 2), "achieved_GBps": round(gbps, 1),
                         "e_lib_pct": round(e_lib, 1) if e_lib is not None else ""})
            print(f"{kernel:<14} {size:<17} {impl:<8} {m['latency_ms']:>11.4f} "
                  f"{m['peak_memory_mb']:>11.2f} {m['device_us']:>10.2f} {gbps:>8.1f} "
                  f"{(e_lib if e_lib is not None else float('nan')):>8.1f}  {desc}", flush=True)
        del dev_args
    return rows


def write_csv(path, rows) -> None:
    with open(path, "w", newline="") as f:
        writer = csv.DictWriter(f, fieldnames=FIELDS)
        writer.writeheader()
        writer.writerows(rows)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default="profile.MI355X.csv")
    ap.add_argument("--kernels", nargs="*", default=None)
    ap.add_argument("--no-configs", action="store_true", help="reference cases only")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    print(f"{'Kernel':<14} {'Size':<17} {'Impl':<8} {'Latency(ms)':>11} {'PeakMem(MB)':>11} "
          f"{'device_us':>10} {'GB/s':>8} {'E_lib%':>8}  Input", flush=True)
    chosen = [c for c in cases(not args.no_configs)
              if not args.kernels or c[0] in args.kernels]
    rows = run_cases(chosen)
    write_csv(args.out, rows)
    print(f"\nResults written to {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
