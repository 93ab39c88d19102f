"""Result formats of the HIP backend (CPU tier).

* the ViperBench-format profile keeps the reference's profile.csv columns first
  (ViperBench/results/profile.GH200-480GB.csv:1) and has a hip row next to every
  pytorch row;
* elib.py computes compute_elib.py's table (experiments/compute_elib.py:49-87):
  E_lib = t_pytorch / t_impl x 100, its columns, and the geomean summary;
* cliff_roofline rows carry exp_cliff_roofline.py's columns (:472-477) after the
  gpu identity columns (_harness.py:192-205), with E_lib_opt = t_lib / t_opt and
  roofline_frac_opt = essential bytes / t_opt / peak.
"""
import csv
import math
from pathlib import Path

import pytest

from dslperfgap_amd import harness

from dslperfgap_amd.viperbench import benchmark, cliff_roofline, elib

RESULTS = Path(__file__).resolve().parents[1] / "dslperfgap_amd" / "viperbench" / "results"
PROFILE_COLUMNS = ["kernel", "size", "impl", "input_desc", "latency_ms", "peak_memory_mb"]
CLIFF_COLUMNS = ["kernel", "dsl", "dtype", "shape", "t_lib_ms", "t_naive_ms", "t_opt_ms",
                 "E_lib_naive", "E_lib_opt", "cliff", "roofline_bound_type",
                 "roofline_peak_assumed", "roofline_frac_opt", "note"]


def test_profile_columns_start_with_the_reference_header():
    assert benchmark.FIELDS[:6] == PROFILE_COLUMNS


def test_committed_profile_has_hip_beside_every_pytorch_row():
    path = RESULTS / "profile.MI355X.csv"
    with open(path, newline="") as f:
        reader = csv.DictReader(f)
        assert reader.fieldnames[:6] == PROFILE_COLUMNS
        rows = list(reader)
    keys = {(r["kernel"], r["size"], r["impl"]) for r in rows}
    torch_rows = {(k, s) for k, s, i in keys if i == "pytorch"}
    assert torch_rows, "no pytorch rows"
    for k, s in torch_rows:
        assert (k, s, "hip") in keys, (k, s)
    for r in rows:
        assert float(r["latency_ms"]) > 0 and float(r["device_us"]) > 0


def test_elib_matches_compute_elib(tmp_path):
    p = tmp_path / "profile.X.csv"
    with open(p, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(PROFILE_COLUMNS)
        w.writerow(["k1", "large", "pytorch", "d", "2.0", "1"])
        w.writerow(["k1", "large", "hip", "d", "0.5", "1"])
        w.writerow(["k1", "small", "pytorch", "d", "1.0", "1"])
        w.writerow(["k1", "small", "hip", "d", "ERROR", "1"])   # skipped like compute_elib
        w.writerow(["k2", "large", "hip", "d", "1.0", "1"])     # no baseline -> no cell
        w.writerow(["k2", "small", "pytorch", "d", "3.0", "1"])
        w.writerow(["k2", "small", "hip", "d", "4.0", "1"])
    rows = list(elib.compute(elib.load(p)))
    assert [(r[0], r[1], r[2]) for r in rows] == [("k1", "large", "hip"), ("k2", "small", "hip")]
    assert rows[0][5] == pytest.approx(400.0)
    assert rows[1][5] == pytest.approx(75.0)
    out = tmp_path / "elib.X.csv"
    assert elib.main([str(p)]) == 0
    with open(out, newline="") as f:
        got = list(csv.reader(f))
    assert got[0] == elib.OUT_FIELDS == ["kernel", "size", "impl", "pytorch_ms", "dsl_ms",
                                         "elib_percent"]
    assert got[1] == ["k1", "large", "hip", "2", "0.5", "400.00"]
    assert elib.geomean([400.0, 25.0]) == pytest.approx(100.0)
    assert math.isnan(elib.geomean([]))


def test_committed_elib_agrees_with_committed_profile():
    want = {(k, s, i): e for k, s, i, _b, _t, e in
            elib.compute(elib.load(RESULTS / "profile.MI355X.csv"))}
    with open(RESULTS / "elib.MI355X.csv", newline="") as f:
        got = {(r["kernel"], r["size"], r["impl"]): float(r["elib_percent"])
               for r in csv.DictReader(f)}
    assert got.keys() == want.keys()
    for key, e in want.items():
        assert got[key] == pytest.approx(e, abs=0.006), key


def test_cliff_row_uses_the_kernels_measured_yardstick():
    peaks = {"copy": 6.6e12, "read": 7.0e12}
    r = cliff_roofline.make_row("logsumexp", 0.5, 0.1, 0.1, 5e8, 8.0e12, "n", peaks)
    assert r["measured_peak"] == "read 7000.0 GB/s"
    assert r["frac_of_measured_peak_hbm"] == pytest.approx(5e8 / 1e-4 / 7.0e12, abs=1e-4)
    r = cliff_roofline.make_row("softmax", 0.5, 0.1, 0.1, 5e8, 8.0e12, "n", peaks)
    assert r["measured_peak"] == "copy 6600.0 GB/s"
    assert harness.peak_kind("cross_entropy") == "read" and harness.peak_kind("rms_norm") == "copy"


def test_cliff_row_format(tmp_path):
    row = cliff_roofline.make_row("rms_norm", 0.5, 0.05, 0.06, 268_451_840, 8.0e12, "n")
    assert list(row)[:14] == CLIFF_COLUMNS
    assert row["dsl"] == "hip" and row["t_naive_ms"] == "" and row["cliff"] == ""
    assert row["E_lib_opt"] == pytest.approx(10.0)
    assert row["roofline_frac_opt"] == pytest.approx(268_451_840 / 0.05e-3 / 8.0e12, abs=1e-4)
    assert row["roofline_frac_opt_hbm"] == pytest.approx(268_451_840 / 0.06e-3 / 8.0e12,
                                                         abs=1e-4)
    out = tmp_path / "s" / "cliff_roofline.csv"
    cliff_roofline.write_rows(out, [row], {"gpu_name": "g", "sm": "gfx950", "timestamp_utc": "t"})
    with open(out, newline="") as f:
        header = next(csv.reader(f))
    assert header[:3] == ["gpu_name", "sm", "timestamp_utc"]
    assert header[3:17] == CLIFF_COLUMNS


def test_cliff_entries_follow_kernel_configs():
    """AKO4ALL/prepare_kernel.py KERNEL_CONFIGS large shapes for the family."""
    want = {"layer_norm": (8192, 8192), "rms_norm": (8192, 8192), "argmax": (8192, 32768),
            "max_reduction": (8192, 32768), "mean_reduction": (8192, 32768),
            "softmax": (4096, 32768), "log_softmax": (4096, 32768),
            "logsumexp": (8192, 16384), "cross_entropy": (4096, 32768)}
    assert set(cliff_roofline.ENTRIES) == set(want)
    for k, shape in want.items():
        assert f"{shape[0]},{shape[1]}" in cliff_roofline.ENTRIES[k][2], k
    assert cliff_roofline.device_slug("AMD Instinct MI355X") == "AMD_Instinct_MI355X"
    assert cliff_roofline.device_slug("AMD Radeon Graphics", "gfx950") == "AMD_gfx950"


def test_committed_cliff_table_is_consistent():
    """One hip row per family kernel; E_lib_opt and the roofline fraction follow
    from the row's own times and the 8 TB/s MI355X figure."""
    path = RESULTS / "AMD_gfx950" / "cliff_roofline.csv"
    with open(path, newline="") as f:
        reader = csv.DictReader(f)
        assert reader.fieldnames[3:17] == CLIFF_COLUMNS
        rows = list(reader)
    assert sorted(r["kernel"] for r in rows) == sorted(cliff_roofline.ENTRIES)
    for r in rows:
        assert r["dsl"] == "hip" and r["sm"] == "gfx950"
        t_lib, t_opt = float(r["t_lib_ms"]), float(r["t_opt_ms"])
        assert float(r["E_lib_opt"]) == pytest.approx(t_lib / t_opt, rel=1e-3)
        work = int(r["note"].split("essential bytes ")[1].split(";")[0])
        assert float(r["roofline_frac_opt"]) == pytest.approx(work / (t_opt * 1e-3) / 8e12,
                                                              abs=2e-4)
        # the measured yardstick fits the kernel: the streaming read for the
        # read-dominated kernels, the copy otherwise; no fraction exceeds it
        kind, rate = r["measured_peak"].split()[:2]
        assert kind == harness.peak_kind(r["kernel"]), r["kernel"]
        t_hbm = float(r["t_opt_hbm_ms"])
        frac = float(r["frac_of_measured_peak_hbm"])
        assert frac == pytest.approx(work / (t_hbm * 1e-3) / (float(rate) * 1e9), rel=2e-3)
        assert 0 < frac <= 1.0, (r["kernel"], frac)


def test_committed_width_scan_is_complete():
    """The row-width scan holds every kernel of width_scan.KERNELS at every
    width of width_scan.WIDTHS once, at about 64 MiB of input per call, with
    hip_over_torch the ratio of its own two rates."""
    import torch

    from dslperfgap_amd.viperbench import width_scan

    path = RESULTS / "AMD_gfx950" / "width_scan.csv"
    with open(path, newline="") as f:
        reader = csv.DictReader(f)
        assert reader.fieldnames == ["kernel", "dtype", "rows", "cols", "hip_GBps", "torch_GBps",
                                     "hip_over_torch"]
        rows = list(reader)
    want = {(k, w) for k, *_ in width_scan.KERNELS for w in width_scan.WIDTHS}
    got = [(r["kernel"], int(r["cols"])) for r in rows]
    assert len(got) == len(set(got)) and set(got) == want
    dtypes = {k: str(dt).replace("torch.", "") for k, _, dt, _ in width_scan.KERNELS}
    for r in rows:
        assert r["dtype"] == dtypes[r["kernel"]]
        elt = torch.empty(0, dtype=getattr(torch, r["dtype"])).element_size()
        assert int(r["rows"]) == max(1, (64 << 20) // (int(r["cols"]) * elt))
        hip, ref = float(r["hip_GBps"]), float(r["torch_GBps"])
        assert 0 < hip < 8000 and 0 < ref < 8000
        assert float(r["hip_over_torch"]) == pytest.approx(hip / ref, rel=2e-3)
