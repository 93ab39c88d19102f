"""Roofline rows for the HIP backend in the reference's cliff_roofline.csv format.

The counterpart of experiments/exp_cliff_roofline.py:299-384 for this family on
one MI355X.  For each kernel of the family at the large shape of
AKO4ALL/prepare_kernel.py's KERNEL_CONFIGS (the shapes exp_cliff_roofline.py
times), it measures

* ``t_lib_ms``  torch's own GPU implementation (``harness.library_fn``), and
* ``t_opt_ms``  the drop-in ``hip_impl`` function,

with the reference's protocol (experiments/_harness.py:110-139: CUDA/HIP events
around single calls, 15 warm-up + 50 timed, median; the same inputs every call),
and writes one row per kernel with the reference's columns
(exp_cliff_roofline.py:472-477, plus gpu_name / sm / timestamp_utc,
_harness.py:192-205).  ``dsl`` is ``hip``; the naive / cliff columns stay
empty because this backend has a single variant.  The roofline anchor is
essential bytes / t_opt against the MI355X HBM figure (``harness.PEAKS``),
with logsumexp and cross_entropy byte models that the reference lacks
(exp_cliff_roofline.py:263).

The reference protocol reuses one input set, so a working set under the 256 MB
Infinity Cache is partly served from it.  Four columns are appended: the
median device time with inputs cycled through >= 2 GiB of HBM copies
(``t_opt_hbm_ms``), the roofline fraction from it (``roofline_frac_opt_hbm``),
the measured yardstick of the kernel (``measured_peak``: the 4 GiB stream copy,
read + write, for kernels that read and write about as much; the 4 GiB
streaming read for logsumexp, cross entropy and mean / max / argmax, which
write almost nothing), and the achieved rate as a fraction of it
(``frac_of_measured_peak_hbm``).

An entry that raises does not end the sweep: as exp_cliff_roofline.py:450-461
does, it gets a row with the measured columns empty and the note
``ENTRY_ERROR: <type>: <message>``, and the next entry runs.

    python -m dslperfgap_amd.viperbench.cliff_roofline [--kernels a,b] [--out PATH]
"""
from __future__ import annotations

import argparse
import csv
import importlib
import re
import sys
from datetime import datetime, timezone
from pathlib import Path

import torch

from dslperfgap_amd import harness
from dslperfgap_amd.viperbench.benchmark import device_time_us
from dslperfgap_amd.workloads import to_device

RESULTS = Path(__file__).resolve().parent / "results"
FIELDS = ["kernel", "dsl", "dtype", "shape", "t_lib_ms", "t_naive_ms", "t_opt_ms",
          "E_lib_naive", "E_lib_opt", "cliff", "roofline_bound_type", "roofline_peak_assumed",
          "roofline_frac_opt", "note", "t_opt_hbm_ms", "roofline_frac_opt_hbm",
          "measured_peak", "frac_of_measured_peak_hbm"]
META = ["gpu_name", "sm", "timestamp_utc"]


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _randn(seed, *shape, dtype=torch.float32):
    return torch.randn(*shape, generator=_g(seed)).to(dtype)


# kernel -> (hip_impl function, dtype label, shape text, input maker, KERNEL_CONFIGS lines)
ENTRIES = {
    "layer_norm": ("layer_norm", "bf16", "x:(8192,8192) w,b:(8192) bf16",
                   lambda: [_randn(1, 8192, 8192, dtype=torch.bfloat16),
                            _randn(2, 8192, dtype=torch.bfloat16),
                            _randn(3, 8192, dtype=torch.bfloat16)], "74-84"),
    "rms_norm": ("rms_norm", "fp16", "x:(8192,8192) w:(8192) fp16",
                 lambda: [_randn(4, 8192, 8192, dtype=torch.float16), (8192,),
                          _randn(5, 8192, dtype=torch.float16)], "85-95"),
    "argmax": ("argmax", "fp16", "x:(8192,32768) dim=1 fp16",
               lambda: [_randn(6, 8192, 32768, dtype=torch.float16), 1], "36-43"),
    "max_reduction": ("max_reduction", "fp16", "x:(8192,32768) dim=1 fp16",
                      lambda: [_randn(7, 8192, 32768, dtype=torch.float16), 1], "44-51"),
    "mean_reduction": ("mean_reduction", "fp32", "x:(8192,32768) dim=1 fp32",
                       lambda: [_randn(8, 8192, 32768), 1], "96-103"),
    "softmax": ("softmax", "fp16", "x:(4096,32768) fp16",
                lambda: [_randn(9, 4096, 32768, dtype=torch.float16)], "112-119"),
    "log_softmax": ("log_softmax", "fp16", "x:(4096,32768) fp16",
                    lambda: [_randn(10, 4096, 32768, dtype=torch.float16)], "158-165"),
    "logsumexp": ("logsumexp", "fp32", "x:(8192,16384) fp32",
                  lambda: [_randn(11, 8192, 16384)], "150-157"),
    "cross_entropy": ("cross_entropy_fwd", "fp32", "logits:(4096,32768) fp32 BLOCK_SIZE=1024",
                      lambda: [_randn(12, 4096, 32768),
                               torch.randint(0, 32768, (4096,), generator=_g(13)),
                               0.0, 1.0, 0.0, -100, 32768, 0, 1024, False, False], "224-233"),
}


def gpu_identity() -> dict:
    props = torch.cuda.get_device_properties(0)
    arch = getattr(props, "gcnArchName", "") or ""
    return {"gpu_name": torch.cuda.get_device_name(0), "sm": arch.split(":")[0],
            "timestamp_utc": datetime.now(timezone.utc).isoformat(timespec="seconds")}


def device_slug(name: str, arch: str = "") -> str:
    """Filesystem-safe GPU tag, as _harness.device_slug (experiments/_harness.py:53-57).
    Where the runtime reports only the generic "AMD Radeon Graphics" (no
    marketing-name table on the host), the ISA name stands in for the model."""
    if arch and "Radeon Graphics" in name:
        name = f"AMD {arch}"
    return re.sub(r"[^A-Za-z0-9._-]+", "_", name).strip("_")


def time_ref_protocol(fn, args, warmup: int = 15, reps: int = 50) -> float:
    """experiments/_harness.py:110-139: median ms of event-bracketed single calls."""
    for _ in range(warmup):
        fn(*args)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn(*args)
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    times.sort()
    return times[len(times) // 2]


def make_row(kernel: str, t_lib: float | None, t_opt: float, t_hbm: float | None,
             work: int, peak: float, peak_note: str, peaks: dict | None = None) -> dict:
    """One cliff_roofline row (times in ms, work in bytes, peak in bytes/s;
    `peaks`: the measured {"copy": ..., "read": ...} rates in bytes/s)."""
    kind = harness.peak_kind(kernel)
    measured = peaks.get(kind) if peaks else None
    _fn, dtype, shape, _make, lines = ENTRIES[kernel]
    frac = work / (t_opt * 1e-3) / peak
    note = (f"hip_impl (gfx950 HIP); shape from AKO4ALL/prepare_kernel.py:{lines}; no naive "
            f"variant | roofline[memory]: essential bytes {work}; "
            f"achieved={work / (t_opt * 1e-3):.3g}B/s; peak={peak:.3g}B/s; {peak_note}")
    return {
        "kernel": kernel, "dsl": "hip", "dtype": dtype, "shape": shape,
        "t_lib_ms": round(t_lib, 5) if t_lib else "", "t_naive_ms": "",
        "t_opt_ms": round(t_opt, 5), "E_lib_naive": "",
        "E_lib_opt": round(t_lib / t_opt, 4) if t_lib else "", "cliff": "",
        "roofline_bound_type": "memory", "roofline_peak_assumed": f"{peak:.4g} B/s HBM (MI355X)",
        "roofline_frac_opt": round(frac, 4), "note": note,
        "t_opt_hbm_ms": round(t_hbm, 5) if t_hbm else "",
        "roofline_frac_opt_hbm": round(work / (t_hbm * 1e-3) / peak, 4) if t_hbm else "",
        "measured_peak": f"{kind} {measured / 1e9:.1f} GB/s" if measured else "",
        "frac_of_measured_peak_hbm":
            round(work / (t_hbm * 1e-3) / measured, 4) if t_hbm and measured else "",
    }


def error_row(kernel: str, err: Exception) -> dict:
    """The row of an entry that raised (exp_cliff_roofline.py:452-461)."""
    _fn, dtype, shape, _make, _lines = ENTRIES[kernel]
    row = {f: "" for f in FIELDS}
    row.update(kernel=kernel, dsl="hip", dtype=dtype, shape=shape,
               note=f"ENTRY_ERROR: {type(err).__name__}: {str(err)[:120]}")
    return row


def measure_entry(kernel: str, warmup: int, reps: int, peak: float, peak_note: str,
                  peaks: dict) -> dict:
    """One entry's row: torch's and the hip impl's times, then the HBM-cycled one."""
    fn_name, _dtype, _shape, make, _lines = ENTRIES[kernel]
    cpu_args = make()
    dev = to_device(cpu_args, "cuda")
    hip = getattr(importlib.import_module(f"dslperfgap_amd.viperbench.{kernel}.hip_impl"),
                  fn_name)
    t_lib = time_ref_protocol(harness.library_fn(kernel), dev, warmup, reps)
    t_opt = time_ref_protocol(hip, dev, warmup, reps)
    work = harness.essential_work(kernel, dev)
    del dev
    torch.cuda.empty_cache()
    t_hbm = device_time_us(hip, cpu_args, work) * 1e-3
    return make_row(kernel, t_lib, t_opt, t_hbm, work, peak, peak_note, peaks)


def run_entries(kernels, measure, log=print) -> list[dict]:
    """measure(kernel) for each kernel; one that raises gets an ENTRY_ERROR row."""
    rows = []
    for kernel in kernels:
        try:
            row = measure(kernel)
        except Exception as e:
            log(f"  [error] {kernel} (hip): {type(e).__name__}: {str(e)[:120]}")
            rows.append(error_row(kernel, e))
        else:
            rows.append(row)
            log(f"{kernel:<15}{row['dtype']:<6}{row['t_lib_ms']:>10}{row['t_opt_ms']:>10}"
                f"{row['E_lib_opt']:>10}{row['roofline_frac_opt']:>10}{row['t_opt_hbm_ms']:>10}"
                f"{row['roofline_frac_opt_hbm']:>10}{row['frac_of_measured_peak_hbm']:>9}")
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
    return rows


def write_rows(path: Path, rows: list[dict], meta: dict) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=META + FIELDS)
        w.writeheader()
        for r in rows:
            w.writerow({**meta, **r})


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--kernels", default=None, help="comma-separated subset")
    ap.add_argument("--out", default=None, help="default: results/<gpu_slug>/cliff_roofline.csv")
    ap.add_argument("--warmup", type=int, default=15)
    ap.add_argument("--reps", type=int, default=50)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 2
    meta = gpu_identity()
    peak, peak_note = harness.select_peak(meta["gpu_name"] + " " + meta["sm"])
    if peak is None:
        print(peak_note, file=sys.stderr)
        return 2
    kernels = args.kernels.split(",") if args.kernels else list(ENTRIES)
    peaks = {"copy": harness.copy_peak("cuda:0"), "read": harness.read_peak("cuda:0")}
    print(f"measured stream-copy rate: {peaks['copy'] / 1e9:.1f} GB/s, streaming read: "
          f"{peaks['read'] / 1e9:.1f} GB/s", flush=True)
    print(f"{'kernel':<15}{'dtype':<6}{'t_lib':>10}{'t_opt':>10}{'E_lib_opt':>10}"
          f"{'roof_opt':>10}{'t_hbm':>10}{'roof_hbm':>10}{'of_meas':>9}", flush=True)
    rows = run_entries(kernels, lambda k: measure_entry(k, args.warmup, args.reps, peak,
                                                        peak_note, peaks),
                       log=lambda m: print(m, flush=True))
    out = Path(args.out) if args.out else RESULTS / device_slug(meta["gpu_name"], meta["sm"]) / \
        "cliff_roofline.csv"
    write_rows(out, rows, meta)
    print(f"results -> {out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
