#!/usr/bin/env python3
"""Benchmark of the MI355X HIP backend for ViperBench's normalization family.

Metric: achieved HBM GB/s per kernel, as a fraction of the
measured MI355X stream-copy peak; latency in microseconds.

A "step" is one launch of the hot-path kernel over one batch of the workload.
BASELINE.json's metric is quoted per kernel, on no single config, so the
default workload is the largest single-GPU config: C4, the cross-entropy
forward over fp32 logits [8192, 32000] (configs[3], 1.05 GB per launch).
Inputs are generated on the CPU with a fixed seed and copied to HBM before
timing; the launches cycle through enough copies (>= 2 GiB in total) that no
launch finds its data in the 256 MB Infinity Cache.  Before the timed region
the kernel runs back to back for 0.5 s (every copy touched, clocks at steady
state), then for W warm-up launches; the K timed launches follow, bracketed by
device events on the launch stream and by a roctx range
``vbh-timed:<workload>:<K>`` that profiles select their dispatches by.
``value`` = algorithmic bytes x K / event time of the timed region.

The headline line also carries ``per_config``: every measured config (C1-C5
and the C4 backward), each timed the same way over its own rotation with
enough launches for about 50 ms of device time (median of 3 such runs), next
to a same-size yardstick (the stream copy, or the streaming read for the
read-only kernels, moving the same bytes per launch through the same >= 2 GiB
rotation) and to the same launches replayed from a HIP graph (no host work
between kernels).  C1 adds the HIP runtime's own device-to-device copy
(hipMemcpyAsync) of its size; C4 adds its full step, the row pass followed by
the scalar mean of the 8192 row losses on the GPU (``full_step``).

  python bench.py [--steps K] [--warmup W] [--workload KEY] [--all] [--no-cpu]
                  [--no-per-config] [--graph] [--copy-at B ...] [--read-at B ...]
                  [--runtime-copy-at B ...]

Prints ONE JSON line on stdout (``--all``: one per workload).  Progress goes
to stderr.  Only one GPU is used: ``--gpus`` above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

import torch

from dslperfgap_amd import _lib, _roctx, harness
from dslperfgap_amd.workloads import HEADLINE, WORKLOADS

METRIC = "achieved HBM GB/s and % of measured MI355X peak per kernel; latency µs"
VENDOR_PEAK_GBPS = 8000.0
TRAFFIC_FILE = Path(__file__).resolve().parent / "profiles" / "row_kernels_all_configs_hbm_traffic.txt"


def measured_traffic(key: str):
    """HBM bytes per launch of workload `key` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by the copy-kernel factors), or None."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 3 and parts[0] == "TRAFFIC" and parts[1] == key:
            fields = dict(p.split("=", 1) for p in parts[2:] if "=" in p)
            return int(fields["bytes_per_launch"])
    return None


def lib_srchash() -> str:
    """First 16 hex digits of the source hash the loaded library was built from
    (checked against the tree by _lib.lib())."""
    p = _lib.LIB_PATH.with_suffix(".srchash")
    return p.read_text().strip()[:16] if p.exists() else None


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(w, cpu_args, budget_s: float) -> dict:
    """Time the oracle's CPU restatement of the reference golden on the same
    inputs, on this host's cores (reported baseline only)."""
    from oracle import pytorch_impl as ref  # the checker doubles as the CPU path

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    fn = getattr(ref, w.fn)
    warm = 1 if w.fn.startswith("cross_entropy") else 3
    for _ in range(warm):
        fn(*cpu_args)
    # timed calls until `budget_s` seconds of CPU work (at least 3 calls)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        fn(*cpu_args)
        times.append(time.perf_counter() - t0)
    total = time.perf_counter() - t_start
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(w.bytes_per_launch / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"full {w.key} shape, oracle restatement of the reference golden "
                   f"(torch CPU), {warm} warm-up + {len(times)} timed calls in {total:.1f} s, "
                   f"median {med * 1e3:.2f} ms; CPU: {cpu_model()}"),
        "ms": round(med * 1e3, 3),
    }


DEVICE_WARM_S = 0.5

# the configs of BASELINE.json (and the C4 backward) in the per_config block
PER_CONFIG = ("C1_layer_norm", "C2_rms_norm", "C3_softmax", "C3_log_softmax", "C3_logsumexp",
              "C4_cross_entropy", "C4_cross_entropy_bwd", "C5_layer_norm")
PER_CONFIG_DEVICE_S = 0.05   # device time of one timed run per config
PER_CONFIG_REPEATS = 3


def timed_rate(launch, nbytes, device_s=PER_CONFIG_DEVICE_S, repeats=PER_CONFIG_REPEATS):
    """Median over `repeats` runs of back-to-back launches (about `device_s`
    of device time each, event-timed, after a 0.3 s warm-up): GB/s and
    microseconds per launch."""
    harness.warm_gpu(launch, 0.3)
    probe = harness.time_back_to_back(launch, 20, 2)["event_ms"] / 20
    n = int(min(5000, max(100, device_s * 1e3 / max(probe, 1e-6))))
    runs = sorted(harness.time_back_to_back(launch, n, 2)["event_ms"] / n for _ in range(repeats))
    ms = runs[len(runs) // 2]
    return {"value": round(nbytes / (ms * 1e-3) / 1e9, 2), "latency_us": round(ms * 1e3, 3),
            "launches": n, "repeats": repeats,
            "latency_us_runs": [round(r * 1e3, 3) for r in runs]}


def yardstick(kind, nbytes):
    """The stream copy (kind "copy": nbytes moved, half read, half written) or
    the streaming read (kind "read") at one launch's byte count, cycling
    through >= 2 GiB."""
    if kind == "read":
        launch, moved, _ = harness.read_rotation("cuda:0", nbytes)
    else:
        launch, moved, _ = harness.copy_rotation("cuda:0", nbytes)
    r = timed_rate(launch, moved)
    del launch
    return {"kind": kind, "bytes": moved, "value": r["value"], "latency_us": r["latency_us"]}


def per_config(peaks) -> dict:
    """One entry per measured config: value, latency, fractions of the vendor
    peak and of the measured peak of its kind, the same-size yardstick and the
    graph-replayed latency; C1 and C4 carry their extra studies."""
    out = {}
    for key in PER_CONFIG:
        w = WORKLOADS[key]
        log(f"[bench] per_config {key}")
        cpu_args = w.make()
        rot = harness.make_rotation(w, cpu_args, "cuda:0")
        n_rows = cpu_args[0].shape[0]
        del cpu_args
        r = timed_rate(rot.launch, w.bytes_per_launch)
        g = harness.graph_replay_ms(rot.launch, rot.copies * max(1, 64 // rot.copies))
        graph_us = g["ms_per_launch"] * 1e3
        y = yardstick(w.peak_kind, w.bytes_per_launch)
        e = {
            "value": r["value"], "unit": "GB/s", "latency_us": r["latency_us"],
            "frac": round(r["value"] / VENDOR_PEAK_GBPS, 4),
            "frac_of_measured_peak": round(r["value"] * 1e9 / peaks[w.peak_kind], 4),
            "peak_kind": w.peak_kind,
            "algorithmic_bytes": w.bytes_per_launch,
            "launches": r["launches"], "repeats": r["repeats"],
            "latency_us_runs": r["latency_us_runs"],
            "graph_replay": {"latency_us": round(graph_us, 3),
                             "value": round(w.bytes_per_launch / (graph_us * 1e-6) / 1e9, 2),
                             "launches_per_graph": g["launches_per_graph"],
                             "replays": g["replays"]},
            "same_size_yardstick": y,
            "frac_of_same_size_yardstick": round(r["value"] / y["value"], 4),
        }
        if key == "C1_layer_norm":
            launch, moved, _ = harness.runtime_copy_rotation("cuda:0", w.bytes_per_launch)
            rc = timed_rate(launch, moved)
            del launch
            e["runtime_copy_same_size"] = {
                "what": "hipMemcpyAsync device-to-device (torch copy_) of "
                        f"{moved // 2} B per launch, >= 2 GiB rotation",
                "value": rc["value"], "latency_us": rc["latency_us"]}
            e["frac_of_runtime_copy_same_size"] = round(r["value"] / rc["value"], 4)
        if key == "C4_cross_entropy":
            launch, scalars = harness.ce_mean_step(rot, n_rows)
            full_bytes = w.bytes_per_launch + n_rows * 4 + 4
            f = timed_rate(launch, full_bytes)
            torch.cuda.synchronize()
            e["full_step"] = {
                "what": "cross_entropy_fwd row pass, then the mean of the 8192 row losses "
                        "(vbh_reduce_fwd) on the same stream",
                "value": f["value"], "latency_us": f["latency_us"],
                "mean_latency_us": round(f["latency_us"] - r["latency_us"], 3),
                "algorithmic_bytes": full_bytes,
                "loss_mean": float(scalars[0].item())}
            del launch, scalars
        out[key] = e
        del rot
        torch.cuda.empty_cache()
    return out


def run_workload(key, steps, warmup, peaks, with_cpu, cpu_budget, graph=False):
    w = WORKLOADS[key]
    log(f"[bench] {key}: generating inputs")
    cpu_args = w.make()
    rot = harness.make_rotation(w, cpu_args, "cuda:0")
    log(f"[bench] {key}: {rot.copies} HBM copies, {w.bytes_per_launch} B per launch")
    # median of single launches (each fenced by its own events), before the
    # timed region so that the timed launches are the workload's last dispatches
    single = harness.time_kernel(rot.launch, reps=50, warmup=5)
    # steady state before timing: 0.5 s of back-to-back launches (clocks, page
    # tables, every HBM copy touched), then the `warmup` launches inside
    # time_back_to_back, then the timed region
    harness.warm_gpu(rot.launch, DEVICE_WARM_S)
    per_graph = 0
    if graph:
        # the launches as replays of a HIP graph of per_graph consecutive
        # launches: no host work between kernels, under a profiler too
        per_graph = rot.copies * max(1, 64 // rot.copies)
        g = harness.capture_graph(rot.launch, per_graph)
        replays = max(1, steps // per_graph)
        steps = replays * per_graph
        r = harness.time_back_to_back(lambda i: g.replay(), replays,
                                      max(1, warmup // per_graph),
                                      fence=_roctx.range_(f"vbh-timed:{key}:{steps}"))
    else:
        r = harness.time_back_to_back(rot.launch, steps, warmup,
                                      fence=_roctx.range_(f"vbh-timed:{key}:{steps}"))
    per_launch_ms = r["event_ms"] / steps
    value = w.bytes_per_launch * steps / (r["event_ms"] * 1e-3) / 1e9
    vendor_peak = VENDOR_PEAK_GBPS
    peak_kind = w.peak_kind
    peak_measured = peaks[peak_kind]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "device_warm_s": DEVICE_WARM_S,
        "ms_per_step": round(r["wall_ms"] / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "accumulate": "f32",
        "data": "synthetic: seeded CPU generator (BASELINE.json config distributions), copied to HBM",
        "config": {"workload": key, "desc": w.desc, "hbm_copies": rot.copies},
        "latency_us": round(per_launch_ms * 1e3, 3),
        "latency_us_single_launch_median": round(single["median_ms"] * 1e3, 3),
        "timing": (f"HIP graph replays of {per_graph} launches" if graph
                   else "back-to-back launches from the host"),
        "roofline": {
            "bound": "hbm",
            "achieved": round(value, 2),
            "peak": vendor_peak,
            "unit": "GB/s",
            "frac": round(value / vendor_peak, 4),
            "traffic": measured_traffic(key),
            "traffic_source": f"rocprofv3 FETCH_SIZE/WRITE_SIZE, {TRAFFIC_FILE.name}",
            "algorithmic_bytes": w.bytes_per_launch,
        },
        "measured_copy_peak_GBps": round(peaks["copy"] / 1e9, 2),
        "measured_read_peak_GBps": round(peaks["read"] / 1e9, 2),
        "measured_peak_kind": peak_kind,
        "frac_of_measured_peak": round(value * 1e9 / peak_measured, 4),
        "timed_range": f"vbh-timed:{key}:{steps}" if _roctx.available() else None,
        "lib_srchash": lib_srchash(),
    }
    del rot
    torch.cuda.empty_cache()
    if with_cpu:
        log(f"[bench] {key}: CPU baseline")
        line["cpu_baseline"] = cpu_baseline(w, cpu_args, cpu_budget)
    return line


def run_copy_at(nbytes, steps, warmup, peaks, kind="copy"):
    """The stream copy moving `nbytes` per launch (half read, half written),
    with kind "read" the streaming read of `nbytes`, or with kind
    "runtime_copy" the HIP runtime's own device-to-device copy
    (hipMemcpyAsync through torch's copy_) moving `nbytes`, rotated through
    >= 2 GiB and timed like a workload: the yardstick of what a kernel of that
    size can reach."""
    if kind == "read":
        launch, moved, copies = harness.read_rotation("cuda:0", nbytes)
        desc = f"vbh_stream_read of {moved} B per launch, {copies} buffers"
    elif kind == "runtime_copy":
        launch, moved, copies = harness.runtime_copy_rotation("cuda:0", nbytes)
        desc = (f"hipMemcpyAsync device-to-device of {moved // 2} B per launch "
                f"(read + write {moved} B), {copies} buffer pairs")
    else:
        launch, moved, copies = harness.copy_rotation("cuda:0", nbytes)
        desc = (f"vbh_stream_copy of {moved // 2} B per launch "
                f"(read + write {moved} B), {copies} buffer pairs")
    key = f"{kind}@{moved}"
    harness.warm_gpu(launch, DEVICE_WARM_S)
    r = harness.time_back_to_back(launch, steps, warmup,
                                  fence=_roctx.range_(f"vbh-timed:{key}:{steps}"))
    value = moved * steps / (r["event_ms"] * 1e-3) / 1e9
    return {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "device_warm_s": DEVICE_WARM_S,
        "ms_per_step": round(r["wall_ms"] / steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u8", "data": "synthetic (constant bytes)",
        "config": {"workload": key, "desc": desc},
        "latency_us": round(r["event_ms"] / steps * 1e3, 3),
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": VENDOR_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(value / VENDOR_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes": moved},
        # a yardstick line: the copy (or read) rate at this size, next to the 4 GiB ones
        "measured_copy_peak_GBps": round(peaks["copy"] / 1e9, 2),
        "measured_read_peak_GBps": round(peaks["read"] / 1e9, 2),
        "timed_range": f"vbh-timed:{key}:{steps}" if _roctx.available() else None,
        "lib_srchash": lib_srchash(),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=None, choices=sorted(WORKLOADS),
                    help=f"default {HEADLINE} (none when only yardsticks are asked for)")
    ap.add_argument("--all", action="store_true", help="every measured workload, one line each")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-per-config", action="store_true",
                    help="leave the per_config block out of the headline line")
    ap.add_argument("--graph", action="store_true",
                    help="time the workloads' launches as replays of a HIP graph of "
                         "consecutive launches (no host work between kernels)")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of timed CPU work for the CPU baseline")
    ap.add_argument("--copy-at", type=int, nargs="+", metavar="BYTES",
                    help="instead of workloads: the stream copy moving BYTES per launch "
                         "(read + write), one line per size")
    ap.add_argument("--read-at", type=int, nargs="+", metavar="BYTES",
                    help="instead of workloads: the streaming read of BYTES per launch, "
                         "one line per size")
    ap.add_argument("--runtime-copy-at", type=int, nargs="+", metavar="BYTES",
                    help="instead of workloads: the HIP runtime's device-to-device copy "
                         "moving BYTES per launch (read + write), one line per size")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this backend is measured on one GPU only; the row kernels would "
              "shard rows across GPUs with no exchange, which no multi-GPU run here "
              "measures. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    _lib.lib()
    log(f"[bench] device: {torch.cuda.get_device_name(0)}")
    peaks = {"copy": harness.copy_peak("cuda:0"), "read": harness.read_peak("cuda:0")}
    log(f"[bench] measured stream-copy peak: {peaks['copy'] / 1e9:.1f} GB/s (read + write), "
        f"stream-read peak: {peaks['read'] / 1e9:.1f} GB/s")
    yardsticks = args.copy_at or args.read_at or args.runtime_copy_at
    for kind, sizes in (("copy", args.copy_at), ("read", args.read_at),
                        ("runtime_copy", args.runtime_copy_at)):
        for nbytes in sizes or []:
            print(json.dumps(run_copy_at(nbytes, args.steps, args.warmup, peaks, kind)),
                  flush=True)
    if yardsticks and not (args.all or args.workload):
        return
    keys = sorted(WORKLOADS) if args.all else [args.workload or HEADLINE]
    for key in keys:
        line = run_workload(key, args.steps, args.warmup, peaks, not args.no_cpu, args.cpu_budget,
                            graph=args.graph)
        if key == HEADLINE and not args.all and not args.no_per_config:
            line["per_config"] = per_config(peaks)
            line["full_step"] = line["per_config"][HEADLINE]["full_step"]
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
