"""Row-width scan: achieved GB/s of the HIP backend and of torch for every
kernel of the family across row widths, at a fixed size per call.

The reference's benchmark times each kernel at two shapes (benchmark.py:143-335).
A backend can be fast there and fall off a cliff at other widths: rows that are
not a multiple of the 16-byte vector (50257, GPT-2's vocabulary), rows too
short for a wave, rows too long for registers, or too few rows for the GPU.
This scan times the hip_impl functions and torch's own GPU implementations
(harness.library_fn) at 18 widths from 64 to 131072 columns, each call over
about `--mib` MiB of input, inputs cycling through several copies, 60
back-to-back calls per point (device events).  GB/s counts each kernel's
algorithmic bytes: inputs read once, full-size outputs written once.

    python -m dslperfgap_amd.viperbench.width_scan --out width_scan.csv

Columns: kernel, dtype, rows, cols, hip_GBps, torch_GBps, hip_over_torch.
"""
from __future__ import annotations

import argparse
import csv
import sys

import torch

from .. import _lib, harness
from .benchmark import _hip_fn

WIDTHS = [64, 100, 128, 255, 256, 512, 1000, 1024, 2048, 3000, 4096, 8192, 10000, 16384,
          32768, 50257, 65536, 131072]

# (kernel, hip_impl function, dtype, full-size output written)
KERNELS = [
    ("layer_norm", "layer_norm", torch.bfloat16, True),
    ("rms_norm", "rms_norm", torch.bfloat16, True),
    ("softmax", "softmax", torch.float16, True),
    ("log_softmax", "log_softmax", torch.float32, True),
    ("logsumexp", "logsumexp", torch.float32, False),
    ("cross_entropy", "cross_entropy_fwd", torch.float32, False),
    ("argmax", "argmax", torch.float16, False),
    ("mean_reduction", "mean_reduction", torch.float32, False),
]


def make_args(kernel: str, rows: int, cols: int, dtype, gen: torch.Generator) -> tuple:
    x = torch.randn(rows, cols, device="cuda", generator=gen).to(dtype)
    if kernel == "layer_norm":
        return (x, torch.randn(cols, device="cuda", generator=gen).to(dtype),
                torch.randn(cols, device="cuda", generator=gen).to(dtype))
    if kernel == "rms_norm":
        return (x, (cols,), torch.randn(cols, device="cuda", generator=gen).to(dtype))
    if kernel == "cross_entropy":
        labels = torch.randint(0, cols, (rows,), device="cuda", generator=gen)
        return (x, labels, 0.0, 1.0, 0.0, -100, cols, 0, 1 << 18, False, False)
    if kernel in ("argmax", "mean_reduction"):
        return (x, 1)
    return (x,)


def rate(fn, sets, nbytes: int, calls: int) -> float:
    launch = lambda k: fn(*sets[k % len(sets)])  # noqa: E731
    harness.warm_gpu(launch, 0.05)
    r = harness.time_back_to_back(launch, calls, 2 * len(sets))
    return nbytes * calls / (r["event_ms"] * 1e-3) / 1e9


def scan(mib: int = 64, copies: int = 6, calls: int = 60, kernels=None, widths=None):
    gen = torch.Generator(device="cuda").manual_seed(31)
    for kernel, fn_name, dtype, full_out in KERNELS:
        if kernels and kernel not in kernels:
            continue
        hip, lib = _hip_fn(kernel, fn_name), harness.library_fn(kernel)
        elt = torch.empty(0, dtype=dtype).element_size()
        for cols in widths or WIDTHS:
            rows = max(1, (mib << 20) // (cols * elt))
            sets = [make_args(kernel, rows, cols, dtype, gen) for _ in range(copies)]
            nbytes = rows * cols * elt * (2 if full_out else 1)
            h = rate(hip, sets, nbytes, calls)
            t = rate(lib, sets, nbytes, calls)
            del sets
            torch.cuda.empty_cache()
            yield dict(kernel=kernel, dtype=str(dtype).replace("torch.", ""), rows=rows, cols=cols,
                       hip_GBps=round(h, 1), torch_GBps=round(t, 1),
                       hip_over_torch=round(h / t, 3))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out", default="width_scan.csv")
    ap.add_argument("--mib", type=int, default=64, help="input MiB per call")
    ap.add_argument("--kernels", nargs="*", default=None)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    _lib.lib()
    fields = ["kernel", "dtype", "rows", "cols", "hip_GBps", "torch_GBps", "hip_over_torch"]
    with open(args.out, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for row in scan(args.mib, kernels=args.kernels):
            w.writerow(row)
            f.flush()
            print(f"{row['kernel']:15s} {row['dtype']:9s} {row['cols']:7d} cols: hip "
                  f"{row['hip_GBps']:7.0f}  torch {row['torch_GBps']:7.0f}  "
                  f"x{row['hip_over_torch']:.2f}", flush=True)
    print(f"results -> {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
