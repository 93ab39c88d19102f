"""Library efficiency (E_lib) table from a ViperBench-format profile CSV.

The counterpart of experiments/compute_elib.py:1-105 for profiles that carry a
``hip`` impl row: E_lib = t_pytorch / t_impl x 100 (compute_elib.py:4-8), from
the ``latency_ms`` column, for every (kernel, size) that has a ``pytorch`` row.
The output CSV has compute_elib's columns (kernel, size, impl, pytorch_ms,
dsl_ms, elib_percent; compute_elib.py:84-87), so the reference's cross-arch
tables (e.g. ViperBench/results/elib.A100-SXM4-40GB.csv) can take an MI355X
file unchanged.  The printed summary is the geomean / min / max per
(impl, size), as compute_elib.py:90-102 prints it.

    python -m dslperfgap_amd.viperbench.elib [profile.csv] [-o elib.csv]
        [--column latency_ms|device_us]

``--column device_us`` computes the same ratio from the device-event column
that the HIP profile adds (inputs cycled through HBM), which separates kernel
time from host dispatch time at the small shapes.
"""
from __future__ import annotations

import argparse
import csv
import math
import os
import sys
from collections import defaultdict
from pathlib import Path

BASELINE = "pytorch"
DEFAULT_PROFILE = Path(__file__).resolve().parent / "results" / "profile.MI355X.csv"
OUT_FIELDS = ["kernel", "size", "impl", "pytorch_ms", "dsl_ms", "elib_percent"]


def load(path, column: str = "latency_ms") -> dict:
    """{(kernel, size, impl): time} from a profile CSV; rows without a number are skipped."""
    out = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            try:
                out[(row["kernel"], row["size"], row["impl"])] = float(row[column])
            except (KeyError, TypeError, ValueError):
                continue
    return out


def compute(times: dict):
    """Yield (kernel, size, impl, t_pytorch, t_impl, elib_pct) for every non-baseline impl."""
    impls = sorted({i for (_k, _s, i) in times if i != BASELINE})
    for kernel, size in sorted({(k, s) for (k, s, _i) in times}):
        base = times.get((kernel, size, BASELINE))
        if base is None:
            continue
        for impl in impls:
            t = times.get((kernel, size, impl))
            if t is None or t <= 0:
                continue
            yield kernel, size, impl, base, t, base / t * 100.0


def geomean(xs) -> float:
    xs = [x for x in xs if x > 0]
    return math.exp(sum(math.log(x) for x in xs) / len(xs)) if xs else float("nan")


def write(rows, path) -> None:
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(OUT_FIELDS)
        for kernel, size, impl, base, t, e in rows:
            w.writerow([kernel, size, impl, f"{base:.6g}", f"{t:.6g}", f"{e:.2f}"])


def summary(rows) -> list[str]:
    by = defaultdict(list)
    for _k, size, impl, _b, _t, e in rows:
        by[(impl, size)].append(e)
    lines = [f"{'impl':<16}{'size':<18}{'n':>4}{'geomean%':>12}{'min%':>10}{'max%':>10}"]
    for impl, size in sorted(by):
        v = by[(impl, size)]
        lines.append(f"{impl:<16}{size:<18}{len(v):>4}{geomean(v):>12.1f}{min(v):>10.1f}"
                     f"{max(v):>10.1f}")
    return lines


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("profile", nargs="?", default=str(DEFAULT_PROFILE))
    ap.add_argument("-o", "--out", default=None,
                    help="output CSV (default: elib.<gpu>.csv beside a profile.<gpu>.csv)")
    ap.add_argument("--column", default="latency_ms", choices=["latency_ms", "device_us"])
    args = ap.parse_args(argv)
    if not os.path.exists(args.profile):
        print(f"profile not found: {args.profile}", file=sys.stderr)
        return 1
    rows = list(compute(load(args.profile, args.column)))
    if not rows:
        print("no E_lib rows (no pytorch baseline rows?)", file=sys.stderr)
        return 1
    out = args.out
    if out is None:
        name = Path(args.profile).name
        tag = name[len("profile."):] if name.startswith("profile.") else name
        out = str(Path(args.profile).with_name("elib." + tag))
    write(rows, out)
    print(f"# E_lib ({args.column}) from {args.profile} -> {out}; {len(rows)} cells")
    print("\n".join(summary(rows)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
