"""Failure records of the harnesses (CPU tier).

The reference records a failing case and keeps going: run_test writes
ERROR / FAIL records into <kernel>.json (ViperBench/test_utils.py:108-132),
benchmark.py writes an ERROR row per failing implementation
(ViperBench/benchmark.py:388-428), exp_cliff_roofline.py an ENTRY_ERROR row
per failing entry (experiments/exp_cliff_roofline.py:450-461).  Here the
failures are forced on the CPU: a hip impl handed CPU tensors raises (the
backend has no CPU fallback), a function returning wrong values fails its
tolerance, and a measurement that raises stands in for a kernel failure.
"""
import csv
import json

import torch

from dslperfgap_amd.viperbench import benchmark, cliff_roofline
from dslperfgap_amd.viperbench import test_utils as tu
from dslperfgap_amd.viperbench.softmax.hip_impl import softmax as hip_softmax
from oracle import pytorch_impl as ref


def _cases():
    g = torch.Generator().manual_seed(1)
    return [{"name": "small_2d", "dtype": torch.float32, "inputs": (torch.randn(4, 8, generator=g),)},
            {"name": "medium_2d", "dtype": torch.float32,
             "inputs": (torch.randn(16, 64, generator=g),)}]


def test_run_test_records_error_fail_and_pass(tmp_path):
    # ERROR: the hip impl refuses CPU tensors with an exception
    ok, rec = tu.run_test("softmax", _cases(), ref.softmax, hip_softmax, loose_tol=True,
                          results_dir=tmp_path)
    assert not ok and rec["overall"] == "FAIL"
    assert [c["status"] for c in rec["test_cases"]] == ["ERROR", "ERROR"]
    assert "GPU tensors" in rec["test_cases"][0]["traceback"]
    on_disk = json.loads((tmp_path / "softmax_hip.json").read_text())
    assert on_disk == rec and on_disk["kernel"] == "softmax_hip"
    assert tu.exit_code(ok) == 1

    # FAIL with max_err: a result off by 1e-3 at fp32 tolerances (1e-5, loose 2e-5)
    def wrong(x):
        return ref.softmax(x) + 1e-3
    ok, rec = tu.run_test("softmax", _cases(), ref.softmax, wrong, loose_tol=True,
                          results_dir=tmp_path)
    assert not ok and [c["status"] for c in rec["test_cases"]] == ["FAIL", "FAIL"]
    assert abs(rec["test_cases"][0]["max_err"] - 1e-3) < 1e-6

    # PASS records carry max_err and time_ms; the file is rewritten
    ok, rec = tu.run_test("softmax", _cases(), ref.softmax, ref.softmax, results_dir=tmp_path)
    assert ok and rec["overall"] == "PASS" and tu.exit_code(ok) == 0
    assert all(c["status"] == "PASS" and c["max_err"] == 0.0 and "time_ms" in c
               for c in rec["test_cases"])
    assert json.loads((tmp_path / "softmax_hip.json").read_text())["overall"] == "PASS"


def test_run_test_mixed_cases_and_per_case_compare(tmp_path):
    """One case erring does not stop the others; a case's own compare
    function (as cross_entropy/test.py's valid-position compare) is used."""
    cases = _cases()
    cases[1]["compare"] = lambda r, t, d, lo: (True, 0.5)
    calls = []

    def flaky(x):
        calls.append(x.shape)
        if x.shape[0] == 4:
            raise RuntimeError("launch failed")
        return x
    ok, rec = tu.run_test("softmax", cases, ref.softmax, flaky, results_dir=None)
    assert calls == [(4, 8), (16, 64)]
    assert [c["status"] for c in rec["test_cases"]] == ["ERROR", "PASS"]
    assert rec["test_cases"][1]["max_err"] == 0.5 and not ok


def test_tolerances_follow_the_reference():
    assert tu.get_tol(torch.float32) == (1e-5, 1e-5)
    assert tu.get_tol(torch.float16) == (1e-3, 1e-3)
    assert tu.get_tol(torch.bfloat16, True) == (2e-2, 2e-2)
    assert tu.get_tol(torch.int64) == (1e-5, 1e-5)
    a = torch.tensor([1.0, float("nan")])
    assert tu.default_compare(a, a.clone(), torch.float32) == (True, 0.0)
    # tuples compare their tensor elements only
    assert tu.default_compare((a, 3), (a.clone(), 4), torch.float32)[0]


def test_benchmark_sweep_keeps_going_after_errors(tmp_path):
    def make_ok():
        return (torch.randn(8, 16),)

    def make_bad():
        raise MemoryError("inputs do not fit")

    case_list = [("softmax", "small", "softmax", "x:(8,16)", make_ok, False),
                 ("softmax", "bad", "softmax", "x:(?)", make_bad, False),
                 ("softmax", "large", "softmax", "x:(8,16)", make_ok, True)]

    def impls(kernel, fn_name):
        return [("pytorch", lambda: "torch"), ("hip", lambda: "hip")]

    def measure(fn, dev_args, cpu_args, traffic, warmup, iters):
        if fn == "hip" and warmup == 10:  # the hip impl of the first case fails
            raise RuntimeError("hipErrorLaunchFailure")
        return {"latency_ms": 0.5, "peak_memory_mb": 1.0, "device_us": 4.0 if fn == "hip" else 8.0}

    rows = benchmark.run_cases(case_list, impls=impls, measure_fn=measure,
                               to_dev=lambda a, d: a)
    got = [(r["size"], r["impl"], r["latency_ms"]) for r in rows]
    assert got == [("small", "pytorch", 0.5), ("small", "hip", "ERROR"),
                   ("bad", "pytorch", "ERROR"), ("bad", "hip", "ERROR"),
                   ("large", "pytorch", 0.5), ("large", "hip", 0.5)]
    assert rows[1]["peak_memory_mb"] == "ERROR" and rows[1]["device_us"] == "ERROR"
    assert rows[-1]["e_lib_pct"] == 200.0
    out = tmp_path / "profile.csv"
    benchmark.write_csv(out, rows)
    with open(out) as f:
        back = list(csv.DictReader(f))
    assert [r["latency_ms"] for r in back] == ["0.5", "ERROR", "ERROR", "ERROR", "0.5", "0.5"]
    assert list(back[0])[:6] == ["kernel", "size", "impl", "input_desc", "latency_ms",
                                 "peak_memory_mb"]


def test_cliff_sweep_keeps_going_after_errors(tmp_path):
    def measure(kernel):
        if kernel == "softmax":
            raise RuntimeError("hipErrorIllegalAddress in softmax_rows")
        return cliff_roofline.make_row(kernel, 0.2, 0.1, 0.1, 10**8, 8e12, "MI355X")

    logged = []
    rows = cliff_roofline.run_entries(["layer_norm", "softmax", "logsumexp"], measure,
                                      log=logged.append)
    assert [r["kernel"] for r in rows] == ["layer_norm", "softmax", "logsumexp"]
    err = rows[1]
    assert err["note"].startswith("ENTRY_ERROR: RuntimeError: hipErrorIllegalAddress")
    assert err["t_opt_ms"] == "" and err["dsl"] == "hip" and err["dtype"] == "fp16"
    assert any("[error] softmax" in m for m in logged)
    out = tmp_path / "cliff.csv"
    cliff_roofline.write_rows(out, rows, {"gpu_name": "x", "sm": "gfx950", "timestamp_utc": "t"})
    with open(out) as f:
        back = list(csv.DictReader(f))
    assert back[1]["note"].startswith("ENTRY_ERROR") and back[2]["t_opt_ms"] == "0.1"
