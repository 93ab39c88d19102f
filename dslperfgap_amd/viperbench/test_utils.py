"""Correctness records of the HIP backend in ViperBench's run_test format.

The counterpart of ViperBench/test_utils.py:12-216 for the hip impls: each
case runs the reference function and the HIP function on the same inputs,
compares them by the reference's rule (float upcast, ``torch.allclose`` with
the per-dtype tolerances of test_utils.py:12-25, doubled with ``loose_tol``;
tuples element by element, test_utils.py:28-49) and records PASS (with
max_err and the HIP call's wall time in ms), FAIL (with max_err) or ERROR
(with the traceback) per case.  The record goes to
``<results_dir>/<kernel>_hip.json`` as ``{"kernel", "overall", "test_cases"}``,
the layout of ViperBench/results/<kernel>[_impl].json (test_utils.py:120-132,
183-193).

Unlike the reference's ``run_test``, which calls ``sys.exit``, :func:`run_test`
returns ``(all_pass, record)``; ``exit_code`` gives the reference's exit status.
The reference function is the caller's: the GPU tests pass the oracle (the
restated golden), so nothing here imports it.
"""
from __future__ import annotations

import json
import time
import traceback
from pathlib import Path
from typing import Callable

import torch

RESULTS_DIR = Path(__file__).resolve().parent / "results"

# ViperBench/test_utils.py:12-16 (atol, rtol); loose_tol doubles both
_TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (1e-3, 1e-3), torch.bfloat16: (1e-2, 1e-2)}


def get_tol(dtype, loose_tol: bool = False) -> tuple[float, float]:
    """(atol, rtol) for `dtype` (fp32 tolerances for any other dtype)."""
    atol, rtol = _TOL.get(dtype, _TOL[torch.float32])
    return (2 * atol, 2 * rtol) if loose_tol else (atol, rtol)


def _pairs(ref_out, out):
    """Output pairs to compare: tuples element by element, tensor pairs only
    (test_utils.py:38-47)."""
    if isinstance(ref_out, (tuple, list)):
        if not isinstance(out, (tuple, list)) or len(out) != len(ref_out):
            raise TypeError(f"expected {len(ref_out)} outputs, got {type(out).__name__}")
        return [(r, o) for r, o in zip(ref_out, out)
                if isinstance(r, torch.Tensor) and isinstance(o, torch.Tensor)]
    return [(ref_out, out)]


def default_compare(ref_out, out, dtype, loose_tol: bool = False) -> tuple[bool, float]:
    """ViperBench/test_utils.py:28-49: every output pair must be allclose on
    float copies (on the CPU here); max_err is the largest absolute
    difference.  One extension: NaN positions that match count as equal
    (``equal_nan``; the reference's cases hold no NaN, so their verdicts do
    not change)."""
    atol, rtol = get_tol(dtype, loose_tol)
    ok, max_err = True, 0.0
    for r, o in _pairs(ref_out, out):
        r = torch.as_tensor(r).detach().float().cpu()
        o = torch.as_tensor(o).detach().float().cpu()
        if r.shape != o.shape:
            return False, float("inf")
        ok &= bool(torch.allclose(o, r, atol=atol, rtol=rtol, equal_nan=True))
        if r.numel():
            both_nan = r.isnan() & o.isnan()
            d = (o - r).abs().masked_fill(both_nan, 0.0)
            max_err = max(max_err, float(d.nan_to_num(float("inf")).max()))
    return ok, max_err


def _call(fn, inputs):
    if isinstance(inputs, dict):
        return fn(**inputs)
    if isinstance(inputs, (list, tuple)):
        return fn(*inputs)
    return fn(inputs)


def run_test(kernel_name: str, test_cases: list[dict], reference_fn: Callable,
             hip_fn: Callable, loose_tol: bool = False,
             compare_fn: Callable | None = None,
             results_dir: Path | str | None = RESULTS_DIR,
             to_device: Callable | None = None) -> tuple[bool, dict]:
    """Run `test_cases` (dicts with "name", "dtype", "inputs": a dict, list or
    single tensor; optionally "compare", that case's own compare function, as
    cross_entropy/test.py:28-58 compares each configuration's valid positions)
    through `reference_fn` and `hip_fn` and record each.

    `to_device`, if given, maps a case's inputs to the HIP function's inputs
    (e.g. CPU tensors to the GPU); the reference function gets them as given.
    Writes ``<results_dir>/<kernel_name>_hip.json`` unless `results_dir` is None.
    """
    cmp = compare_fn or default_compare
    all_pass, records = True, []
    print(f"\n{'=' * 60}\n  Kernel (HIP): {kernel_name}\n{'=' * 60}", flush=True)
    for tc in test_cases:
        label, dtype, inputs = tc["name"], tc["dtype"], tc["inputs"]
        try:
            ref_out = _call(reference_fn, inputs)
            dev_inputs = to_device(inputs) if to_device else inputs
            if torch.cuda.is_available():
                torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = _call(hip_fn, dev_inputs)
            if torch.cuda.is_available():
                torch.cuda.synchronize()
            elapsed_ms = (time.perf_counter() - t0) * 1000
            passed, max_err = tc.get("compare", cmp)(ref_out, out, dtype, loose_tol)
            if passed:
                print(f"  PASS  {label}  |  max_err={max_err:.2e}  time={elapsed_ms:.2f}ms",
                      flush=True)
                records.append({"name": label, "status": "PASS", "max_err": max_err,
                                "time_ms": elapsed_ms})
            else:
                print(f"  FAIL  {label}  |  max_err={max_err:.2e}  "
                      f"tol={get_tol(dtype, loose_tol)}", flush=True)
                all_pass = False
                records.append({"name": label, "status": "FAIL", "max_err": max_err})
        except Exception:
            tb = traceback.format_exc()
            print(f"  ERROR {label}\n{tb}", flush=True)
            all_pass = False
            records.append({"name": label, "status": "ERROR", "traceback": tb})
    result = {"kernel": f"{kernel_name}_hip", "overall": "PASS" if all_pass else "FAIL",
              "test_cases": records}
    if results_dir is not None:
        out_path = Path(results_dir) / f"{kernel_name}_hip.json"
        out_path.parent.mkdir(parents=True, exist_ok=True)
        out_path.write_text(json.dumps(result, indent=2))
        print(f"\nResult: {result['overall']}  -> {out_path}", flush=True)
    return all_pass, result


def exit_code(all_pass: bool) -> int:
    """The reference's exit status (test_utils.py:132): 0 if every case passed."""
    return 0 if all_pass else 1
