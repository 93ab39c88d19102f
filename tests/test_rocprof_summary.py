"""rocprofv3 summaries (CPU tier): the arithmetic of
dslperfgap_amd/viperbench/rocprof_summary.py on small synthetic CSV files in
rocprofv3's column layout, and the committed summaries that bench.py reads.

* achieved GB/s = algorithmic bytes / AverageNs, of_peak against the kernel's
  measured yardstick of the same run (the 4 GiB copy, or the 4 GiB streaming
  read for the kernels that write almost nothing);
* traffic = (FETCH_SIZE * fetch scale + WRITE_SIZE * write scale) * 1024 with
  the scales set by what the counters read for the copy kernel (4 GiB each way);
* the headers name the directories and prefixes the inputs came from;
* bench.py's roofline.traffic parser reads every config from the committed file.
"""
import csv
import importlib.util
from pathlib import Path

import pytest

from dslperfgap_amd.viperbench import rocprof_summary as rs
from dslperfgap_amd.workloads import WORKLOADS

ROOT = Path(__file__).resolve().parents[1]
C2 = "_ZN3vbh12_GLOBAL__N_113rms_norm_rowsIDF16bDF16bLi8ELi2ELi2EEEvPKT_PKT0_PS2_liif"
COPYK = "vbh::(anonymous namespace)::copy_kernel(unsigned int __vector(4) const*, unsigned int __vector(4)*, long)"
OTHER = "void at::native::reduce_kernel<512, 1>(...)"


def _write(path, header, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)
    return path


def _fixture(tmp_path):
    stats = _write(tmp_path / "run" / "trace" / "all_kernel_stats.csv",
                   ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs",
                    "StdDev"],
                   [[C2, 10, 240000, 24000, 1, 23000, 25000, 100],
                    [COPYK, 2, 2600000, 1300000, 1, 1290000, 1310000, 10],
                    [OTHER, 5, 50, 10, 0, 9, 11, 1]])
    hdr = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    fetch = _write(tmp_path / "run" / "fetch" / "all_counter_collection.csv", hdr,
                   [[1, 1, C2, "FETCH_SIZE", 32768.0], [2, 2, C2, "FETCH_SIZE", 32770.0],
                    [3, 3, COPYK, "FETCH_SIZE", 2097152.0], [4, 4, OTHER, "FETCH_SIZE", 7.0]])
    write = _write(tmp_path / "run" / "write" / "all_counter_collection.csv", hdr,
                   [[1, 1, C2, "WRITE_SIZE", 65536.0], [2, 2, C2, "WRITE_SIZE", 65536.0],
                    [3, 3, COPYK, "WRITE_SIZE", 4194304.0]])
    return stats, fetch, write


def test_trace_and_traffic_arithmetic(tmp_path):
    stats, fetch, write = _fixture(tmp_path)
    alg = rs.config_bytes()
    order = [k for k, _ in rs.CONFIG_KERNELS]
    tr = {r["workload"]: r for r in rs.trace_table(rs.read_stats(stats, rs.CONFIG_KERNELS), alg,
                                                     order)}
    assert set(tr) == {"C2_rms_norm", rs.COPY}
    c2 = tr["C2_rms_norm"]
    assert c2["gbps"] == pytest.approx(134_225_920 / 24000)
    assert c2["peak"] == "copy"
    assert c2["of_peak"] == pytest.approx((134_225_920 / 24000) / (8 * 2**30 / 1_300_000))
    rows, fs, ws = rs.traffic_table(rs.read_counter(fetch, rs.CONFIG_KERNELS),
                                    rs.read_counter(write, rs.CONFIG_KERNELS), alg, order)
    assert fs == pytest.approx(2.0) and ws == pytest.approx(1.0)  # copy reads 2 GiB / 4 GiB
    t = {r["workload"]: r for r in rows}["C2_rms_norm"]
    assert t["dispatches"] == 2 and t["fetch_kib"] == pytest.approx(32769.0)
    assert t["traffic"] == pytest.approx((32769.0 * 2 + 65536.0) * 1024)
    assert t["ratio"] == pytest.approx(t["traffic"] / 134_225_920)


# a symbol of every config's kernel as rocprofv3 printed them
CONFIG_SYMBOLS = {
    "C1_layer_norm": "void vbh::(anonymous namespace)::layer_norm_pipe<float, float, 4, 2, 1, "
                     "false>(float const*, float const*, float const*, float*, long, int, int, "
                     "float)",
    "C3_log_softmax": "void vbh::(anonymous namespace)::softmax_rows<float, float, 4, 2, true, "
                      "2, false>(float const*, float*, long, int, int)",
    "C3_softmax": "void vbh::(anonymous namespace)::softmax_rows<float, float, 4, 2, false, 2, "
                  "false>(float const*, float*, long, int, int)",
    "C3_logsumexp": "void vbh::(anonymous namespace)::logsumexp_rows<float, float, 4, 8, true, "
                    "false>(float const*, float*, long, int, int, int, int)",
    "C4_cross_entropy": "void vbh::(anonymous namespace)::ce_fwd_persist<false, long, true, 256>"
                        "(float const*, long const*, float*, float*, float*, long, int, long)",
    "C4_cross_entropy_bwd": "void vbh::(anonymous namespace)::ce_bwd_tiles<float, 4, 2, false>"
                            "(float const*, float const*, float const*)",
    "C5_layer_norm": "_ZN3vbh12_GLOBAL__N_115layer_norm_pipeIDF16bDF16bLi8ELi4ELi2ELb1EEEvPKT_"
                     "PKT0_S7_PS2_liif",
}


def _full_fixture(tmp_path):
    """The C2 fixture plus one kernel of every other config."""
    stats, fetch, write = _fixture(tmp_path)
    for path, rows in ((stats, [[n, 4, 400, 100, 0, 90, 110, 1] for n in CONFIG_SYMBOLS.values()]),
                       (fetch, [[9, 9, n, "FETCH_SIZE", 100.0] for n in CONFIG_SYMBOLS.values()]),
                       (write, [[9, 9, n, "WRITE_SIZE", 100.0] for n in CONFIG_SYMBOLS.values()])):
        with open(path, "a", newline="") as f:
            csv.writer(f).writerows(rows)
    return stats, fetch, write


READK = "void vbh::(anonymous namespace)::read_kernel<4>(unsigned int __vector(4) const*, unsigned int*, long)"


def test_read_dominated_kernels_use_the_read_yardstick(tmp_path):
    stats = _write(tmp_path / "s.csv",
                   ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs",
                    "StdDev"],
                   [[CONFIG_SYMBOLS["C4_cross_entropy"], 10, 1, 150000, 1, 1, 1, 1],
                    [C2, 10, 240000, 24000, 1, 23000, 25000, 100],
                    [COPYK, 2, 2600000, 1300000, 1, 1290000, 1310000, 10],
                    [READK, 2, 1, 600000, 1, 1, 1, 1]])
    tr = {r["workload"]: r for r in rs.trace_table(rs.read_stats(stats, rs.CONFIG_KERNELS),
                                                     rs.config_bytes(),
                                                     [k for k, _ in rs.CONFIG_KERNELS])}
    c4 = tr["C4_cross_entropy"]
    assert c4["peak"] == "read"
    assert c4["of_peak"] == pytest.approx((1_048_739_840 / 150000) / ((4 << 30) / 600000))
    assert tr[rs.READ]["of_peak"] == pytest.approx(1.0)
    assert tr["C2_rms_norm"]["peak"] == "copy"


def test_every_config_symbol_is_recognised():
    for key, name in CONFIG_SYMBOLS.items():
        assert rs.classify(name, rs.CONFIG_KERNELS) == key, key


def test_a_workload_without_a_kernel_is_an_error(tmp_path):
    """A renamed kernel template must not silently drop a workload (bench.py
    reads the traffic lines)."""
    stats, fetch, write = _fixture(tmp_path)
    with pytest.raises(ValueError, match="C1_layer_norm"):
        rs.render("configs", stats, fetch, write)


def test_rendered_headers_and_machine_lines(tmp_path):
    stats, fetch, write = _full_fixture(tmp_path)
    trace_txt, traffic_txt = rs.render("configs", stats, fetch, write)
    assert f"-d {stats.parent} -o all -- " in trace_txt
    assert f"--pmc FETCH_SIZE --output-format csv -d {fetch.parent} -o all" in traffic_txt
    assert f"--pmc WRITE_SIZE --output-format csv -d {write.parent} -o all" in traffic_txt
    line = [l for l in traffic_txt.splitlines() if l.startswith("TRAFFIC C2_rms_norm")][0]
    assert f"bytes_per_launch={(32769.0 * 2 + 65536.0) * 1024:.0f}" in line
    assert not any("stream_copy" in l for l in traffic_txt.splitlines() if l.startswith("TRAFFIC"))


def test_reference_bytes_match_the_cliff_models():
    b = rs.reference_bytes()
    assert b["layer_norm"] == 2 * 8192 * 8192 * 2 + 2 * 8192 * 2
    assert b["rms_norm"] == 2 * 8192 * 8192 * 2 + 8192 * 2
    assert b["softmax"] == b["log_softmax"] == 2 * 4096 * 32768 * 2
    assert b["logsumexp"] == 8192 * 16384 * 4 + 8192 * 4
    assert b["cross_entropy"] == 4096 * 32768 * 4 + 4096 * 8 + 3 * 4 * 4096 * 32
    assert b["argmax"] == 8192 * 32768 * 2 + 8192 * 8
    assert b["max_reduction"] == 8192 * 32768 * 2 + 8192 * (8 + 2)
    assert b["mean_reduction"] == 8192 * 32768 * 4 + 8192 * 4


def test_bench_reads_traffic_of_every_config_from_the_committed_summary():
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for key, w in WORKLOADS.items():
        t = bench.measured_traffic(key)
        assert t is not None, key
        assert 0.99 < t / w.bytes_per_launch < 1.01, (key, t)


# ---------------------------------------------------------------------------
# timed mode: dispatches inside bench.py's roctx range only
# ---------------------------------------------------------------------------
CE = ("void vbh::(anonymous namespace)::ce_fwd_persist<false, long, true, 256>"
      "(float const*, long const*, float*, float*, float*, long, int, long)")


def _timed_fixture(tmp_path, steps=4):
    kt_hdr = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id",
              "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
    rows, t, did = [], 1000, 0

    def disp(name, dur, gap=1000):
        nonlocal t, did
        did += 1
        rows.append(["KERNEL_DISPATCH", "Agent 1", 1, 0, 1, did, 7, name, did, t, t + dur])
        t += dur + gap

    for _ in range(3):             # warm-up: long launches that must not count
        disp(CE, 900_000)
    start = t - 500
    for i in range(steps):         # timed launches: 150, 160, 170, 180 us
        disp(CE, 150_000 + 10_000 * i)
    disp(OTHER, 10)                # a stray kernel inside the range, not the dominant one
    end = t + 500
    disp(CE, 900_000)              # after the range
    kt = _write(tmp_path / "run" / "c4" / "c4_kernel_trace.csv", kt_hdr, rows)
    mk = _write(tmp_path / "run" / "c4" / "c4_marker_api_trace.csv",
                ["Domain", "Function", "Process_Id", "Thread_Id", "Correlation_Id",
                 "Start_Timestamp", "End_Timestamp"],
                [["MARKER_CORE_RANGE_API", "unrelated", 1, 1, 1, 0, 10**12],
                 ["MARKER_CORE_RANGE_API", f"vbh-timed:C4_cross_entropy:{steps}", 1, 1, 2, start,
                  end]])
    span = rows[3 + steps - 1][10] - rows[3][9]
    line = {"config": {"workload": "C4_cross_entropy"}, "value": 1.0,
            "latency_us": span / steps / 1e3, "roofline": {"frac": 0.5},
            "measured_peak_kind": "read", "frac_of_measured_peak": 0.9}
    bl = tmp_path / "run" / "c4_line.jsonl"
    bl.write_text("progress text\n" + __import__("json").dumps(line) + "\n")
    return kt, mk, bl, span


def test_timed_summary_counts_only_the_timed_dispatches(tmp_path):
    kt, mk, bl, span = _timed_fixture(tmp_path)
    combined, per = rs.render_timed(kt, mk, bl)
    (name, txt), = per.values()
    assert name == "ce_fwd_persist_C4_cross_entropy_timed_trace.txt"
    row = rs.timed_row(rs.read_dispatches(kt), rs.read_ranges(mk)[0],
                       WORKLOADS["C4_cross_entropy"].bytes_per_launch)
    assert row["calls"] == 4 and row["others"] == 1
    assert row["avg_ns"] == pytest.approx(165_000)
    assert row["min_ns"] == 150_000 and row["max_ns"] == 180_000
    assert row["period_ns"] == pytest.approx(span / 4)
    assert row["gbps"] == pytest.approx(1_048_739_840 / 165_000)
    # the bench line's latency equals span / steps here, so they agree exactly
    assert " 1.0000" in txt
    assert f"-d {kt.parent} -o c4 -- " in combined


def test_timed_summary_needs_the_range(tmp_path):
    kt, mk, bl, _ = _timed_fixture(tmp_path)
    empty = _write(tmp_path / "m2.csv", ["Domain", "Function", "Start_Timestamp",
                                         "End_Timestamp"], [])
    with pytest.raises(ValueError, match="no vbh-timed"):
        rs.render_timed(kt, empty, bl)


def test_counter_tail_keeps_the_last_dispatches(tmp_path):
    hdr = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    f = _write(tmp_path / "c.csv", hdr,
               [[i, i, C2, "FETCH_SIZE", 1000.0 if i < 5 else 10.0] for i in range(1, 9)]
               + [[9, 9, COPYK, "FETCH_SIZE", 4.0], [10, 10, COPYK, "FETCH_SIZE", 6.0]])
    all_ = rs.read_counter(f, rs.CONFIG_KERNELS)
    tail = rs.read_counter(f, rs.CONFIG_KERNELS, tail=3)
    assert all_["C2_rms_norm"] == (pytest.approx((4 * 1000 + 4 * 10) / 8), 8)
    assert tail["C2_rms_norm"] == (pytest.approx(10.0), 3)
    assert tail[rs.COPY] == (pytest.approx(5.0), 2)   # the copy kernel keeps every dispatch


def test_kernel_base_names():
    assert rs.kernel_base(CE) == "ce_fwd_persist"
    assert rs.kernel_base(C2) == "rms_norm_rows"
    assert rs.kernel_base(COPYK) == "copy_kernel"
    assert rs.kernel_base(CONFIG_SYMBOLS["C5_layer_norm"]) == "layer_norm_pipe"
    assert rs.timed_file("copy@33562624", COPYK) == "copy_kernel_copy_33562624_timed_trace.txt"
    assert rs.alg_bytes_of("copy@33562624") == 33562624
    assert rs.alg_bytes_of("read@268500992") == 268500992
    assert rs.alg_bytes_of("C1_layer_norm") == WORKLOADS["C1_layer_norm"].bytes_per_launch


def test_instruction_counters_per_wave_and_floor(tmp_path):
    """pipes: per-wave figures divide by SQ_WAVES, VALU/64el by the input's
    elements / 64, the VALU floor is SQ_INSTS_VALU x 4 cycles over 1024 SIMDs at
    2.4 GHz; a counter in two files comes from the first, and --tail keeps the
    last dispatches."""
    hdr = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    a = _write(tmp_path / "a" / "all_counter_collection.csv", hdr,
               [[1, 1, C2, "SQ_WAVES", 999.0], [1, 1, C2, "SQ_INSTS_VALU", 1.0],
                [2, 2, C2, "SQ_WAVES", 8192.0], [2, 2, C2, "SQ_INSTS_VALU", 8192 * 300.0],
                [2, 2, C2, "VALUBusy", 41.5]])
    b = _write(tmp_path / "b" / "all_counter_collection.csv", hdr,
               [[2, 2, C2, "SQ_WAVES", 1.0], [2, 2, C2, "SQ_INSTS_SALU", 8192 * 20.0],
                [2, 2, C2, "SQ_INSTS_VMEM_RD", 8192 * 16.0]])
    c = rs.read_counters([a, b], rs.CONFIG_KERNELS, tail=1)
    assert c["C2_rms_norm"]["SQ_WAVES"] == 8192.0          # from the first file, last dispatch
    stats = {"C2_rms_norm": (C2, 10, 24000.0, 23000.0, 25000.0)}
    (row,) = rs.pipes_table(c, stats, rs.config_elements(), ["C2_rms_norm"])
    assert row["per_wave"]["SQ_INSTS_VALU"] == pytest.approx(300.0)
    assert row["per_wave"]["SQ_INSTS_SALU"] == pytest.approx(20.0)
    assert row["per_wave"]["SQ_INSTS_VMEM_RD"] == pytest.approx(16.0)
    assert row["valu_per_64"] == pytest.approx(8192 * 300.0 / (8192 * 4096 / 64))
    floor = 8192 * 300.0 * 4 / 1024 / 2.4e9 * 1e9
    assert row["valu_floor_ns"] == pytest.approx(floor)
    assert row["floor_share"] == pytest.approx(floor / 24000.0)
    assert row["valu_busy"] == pytest.approx(41.5)


def test_instruction_counters_need_every_config(tmp_path):
    stats, _, _ = _fixture(tmp_path)
    hdr = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    a = _write(tmp_path / "a" / "all_counter_collection.csv", hdr,
               [[2, 2, C2, "SQ_WAVES", 8192.0], [3, 3, COPYK, "SQ_WAVES", 1.0]])
    with pytest.raises(ValueError, match="C1_layer_norm"):
        rs.render_pipes(stats, [a], tail=50)
