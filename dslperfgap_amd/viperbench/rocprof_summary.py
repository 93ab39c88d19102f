"""Text summaries of rocprofv3 output for the HIP backend's kernels.

Reads what ``rocprofv3 --kernel-trace --stats --output-format csv`` writes
(``<prefix>_kernel_stats.csv``) and what ``rocprofv3 --pmc FETCH_SIZE`` /
``--pmc WRITE_SIZE --output-format csv`` write (``<prefix>_counter_collection.csv``),
maps kernel symbols to workloads, and reports per workload:

* calls, average / min / max duration, achieved GB/s = algorithmic bytes /
  average duration, and that rate over the copy kernel's rate in the same run;
* FETCH_SIZE and WRITE_SIZE (KiB per dispatch, averaged over dispatches),
  each scaled by what the counter reads for the 4 GiB copy kernel
  (vbh_stream_copy: 4 GiB read and 4 GiB written per dispatch) in the same
  run, and the ratio of that traffic to the algorithmic bytes -- one read and
  one write of every byte shows as 1.00.

Algorithmic bytes follow the essential-work rule of
experiments/exp_cliff_roofline.py:229-263 (``harness.essential_work``, which
adds logsumexp and cross-entropy byte models), evaluated on meta tensors.

Presets:
  configs    the five measured configs of ``bench.py --all`` (C1-C5)
  reference  the family at the reference's large shapes (cliff_roofline.py)
  pipes      instruction counters (SQ_INSTS_*, SQ_WAVES, VALUBusy) of the
             configs (one or more ``--pmc`` runs of ``bench.py --all``) or,
             with ``--of reference``, of the reference's large shapes (runs of
             cliff_roofline.py)
  timed      the kernel dispatches inside bench.py's timed roctx ranges
             (``vbh-timed:<workload>:<steps>``) next to the lines bench.py
             printed in the same run, whose per-launch event time the traced
             period must agree with -- the headline (bench.py's default run,
             C4), every config, or the copy / read / runtime-copy yardsticks

    python -m dslperfgap_amd.viperbench.rocprof_summary configs \\
        --trace D/trace/all_kernel_stats.csv --fetch D/fetch/all_counter_collection.csv \\
        --write D/write/all_counter_collection.csv --out-dir profiles

    python -m dslperfgap_amd.viperbench.rocprof_summary timed \\
        --kernel-trace D/c4/c4_kernel_trace.csv --markers D/c4/c4_marker_api_trace.csv \\
        --bench-lines D/c4_bench.jsonl --out-dir profiles
"""
from __future__ import annotations

import argparse
import collections
import csv
import re
import sys
from pathlib import Path

import torch

from dslperfgap_amd import harness
from dslperfgap_amd.workloads import WORKLOADS

COPY = "stream_copy_4GiB"
COPY_BYTES = 2 * (4 << 30)         # read + written by one 4 GiB copy dispatch
READ = "stream_read_4GiB"
READ_BYTES = 4 << 30               # read by one 4 GiB streaming-read dispatch
YARDSTICKS = (COPY, READ)
COPY_KIB_EACH_WAY = (4 << 30) // 1024

# workload -> symbol patterns (demangled or mangled; rocprofv3 prints either).
# The row kernels carry their output store policy as an int template argument
# (0 cached, 1 nontemporal, 2 write-through), matched as any digit.
CONFIG_KERNELS = [
    ("C1_layer_norm", r"layer_norm_pipe<float, float, 4, 2, \d, false>|"
                      r"layer_norm_pipeIffLi4ELi2ELi\dELb0E"),
    ("C2_rms_norm", r"rms_norm_rowsIDF16bDF16bLi8ELi2ELi\dE"),
    ("C3_log_softmax", r"softmax_rows<float, float, 4, 2, true, \d(, false)?>"),
    ("C3_softmax", r"softmax_rows<float, float, 4, 2, false, \d(, false)?>"),
    ("C3_logsumexp", r"logsumexp_rows<float, float, 4, 8, true(, false){0,2}>|"
                     r"logsumexp_rowsIffLi4ELi8ELb1E(Lb0E){0,2}E"),
    ("C4_cross_entropy", r"ce_fwd_persist<false, long, true, 256>|ce_fwd_persistILb0ElLb1ELi256EE"),
    ("C4_cross_entropy_bwd", r"ce_bwd_tiles<float, 4, \d(, false)?>|ce_bwd_tilesIfLi4ELi\dE"),
    ("C5_layer_norm", r"layer_norm_pipeIDF16bDF16bLi8ELi4ELi\dELb1E"),
    (COPY, r"copy_kernel\("),
    (READ, r"read_kernel<|read_kernelILi"),
]
REFERENCE_KERNELS = [
    ("layer_norm", r"layer_norm_pipeIDF16bDF16bLi8ELi4ELi\dELb1E"),
    ("rms_norm", r"rms_norm_pipeIDF16_DF16_Li8ELi2ELi\dELb1E"),
    ("softmax", r"softmax_rowsIDF16_DF16_Li8ELi4ELb0ELi\dE"),
    ("log_softmax", r"softmax_rowsIDF16_DF16_Li8ELi4ELb1ELi\dE"),
    ("logsumexp", r"logsumexp_rows<float, float, 4, 8, true(, false){0,2}>|"
                  r"logsumexp_rowsIffLi4ELi8ELb1E(Lb0E){0,2}E"),
    ("cross_entropy", r"ce_fwd_rows<float, 4, \d, true(, false){0,2}>|"
                      r"ce_fwd_rowsIfLi4ELi\dELb1E(Lb0E){0,2}E"),
    ("argmax", r"reduce_rowsIDF16_DF16_Li8ELi2E"),
    ("max_reduction", r"reduce_rowsIDF16_DF16_Li8ELi1E"),
    ("mean_reduction", r"reduce_rows<float, float, 4, 0(, false)?>"),
    (COPY, r"copy_kernel\("),
    (READ, r"read_kernel<|read_kernelILi"),
]


def _meta(shape, dtype=torch.float32):
    return torch.empty(shape, dtype=dtype, device="meta")


def reference_bytes() -> dict:
    """Essential bytes of the reference's large shapes (AKO4ALL/prepare_kernel.py
    KERNEL_CONFIGS, as timed by cliff_roofline.py)."""
    bf, hf = torch.bfloat16, torch.float16
    sq, wide = (8192, 8192), (8192, 32768)
    ew = harness.essential_work
    return {
        "layer_norm": ew("layer_norm", [_meta(sq, bf), _meta((8192,), bf), _meta((8192,), bf)]),
        "rms_norm": ew("rms_norm", [_meta(sq, hf), (8192,), _meta((8192,), hf)]),
        "softmax": ew("softmax", [_meta((4096, 32768), hf)]),
        "log_softmax": ew("log_softmax", [_meta((4096, 32768), hf)]),
        "logsumexp": ew("logsumexp", [_meta((8192, 16384))]),
        "cross_entropy": ew("cross_entropy", [_meta((4096, 32768)), _meta((4096,), torch.int64),
                                              0.0, 1.0, 0.0, -100, 32768, 0, 1024, False, False]),
        "argmax": ew("argmax", [_meta(wide, hf), 1]),
        "max_reduction": ew("max_reduction", [_meta(wide, hf), 1]),
        "mean_reduction": ew("mean_reduction", [_meta(wide), 1]),
        COPY: COPY_BYTES,
        READ: READ_BYTES,
    }


def config_bytes() -> dict:
    out = {k: w.bytes_per_launch for k, w in WORKLOADS.items()}
    out[COPY] = COPY_BYTES
    out[READ] = READ_BYTES
    return out


def classify(name: str, kernels) -> str | None:
    for key, rx in kernels:
        if re.search(rx, name):
            return key
    return None


def read_stats(path, kernels) -> dict:
    """{workload: (symbol, calls, avg_ns, min_ns, max_ns)} from a kernel_stats.csv."""
    out = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            key = classify(r["Name"], kernels)
            if key:
                out[key] = (r["Name"], int(r["Calls"]), float(r["AverageNs"]), float(r["MinNs"]),
                            float(r["MaxNs"]))
    return out


def read_counter(path, kernels, tail: int = 0) -> dict:
    """{workload: (mean counter value per dispatch, dispatches)} from a
    counter_collection.csv; with `tail`, over the last `tail` dispatches of
    each workload's kernel only (the copy kernel always over all of them)."""
    acc = collections.defaultdict(lambda: collections.defaultdict(float))
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            key = classify(r["Kernel_Name"], kernels)
            if key:
                acc[key][int(r["Dispatch_Id"])] += float(r["Counter_Value"])
    out = {}
    for k, per in acc.items():
        ids = sorted(per)
        if tail and k != COPY:
            ids = ids[-tail:]
        out[k] = (sum(per[i] for i in ids) / len(ids), len(ids))
    return out


def peak_kind_of(key: str) -> str:
    """The measured yardstick of a workload or reference kernel: "read" for the
    kernels that write almost nothing, else "copy" (the yardsticks themselves
    are measured against their own kind)."""
    if key == READ:
        return "read"
    if key == COPY:
        return "copy"
    if key in WORKLOADS:
        return WORKLOADS[key].peak_kind
    return harness.peak_kind(key)


def trace_table(stats: dict, alg: dict, order) -> list[dict]:
    rates = {kind: alg[y] / stats[y][2] for kind, y in (("copy", COPY), ("read", READ))
             if y in stats}
    rows = []
    for key in order:
        if key not in stats:
            continue
        name, calls, avg, mn, mx = stats[key]
        gbs = alg[key] / avg
        kind = peak_kind_of(key)
        rows.append(dict(workload=key, kernel=name, calls=calls, avg_ns=avg, min_ns=mn,
                         max_ns=mx, alg_bytes=alg[key], gbps=gbs, peak=kind,
                         of_peak=gbs / rates[kind] if kind in rates else float("nan")))
    return rows


def traffic_table(fetch: dict, write: dict, alg: dict, order):
    """(rows, fetch scale, write scale); scales from the copy kernel of the same runs."""
    fs = COPY_KIB_EACH_WAY / fetch[COPY][0]
    ws = COPY_KIB_EACH_WAY / write[COPY][0]
    rows = []
    for key in order:
        if key not in fetch or key not in write:
            continue
        f_kib, n = fetch[key]
        w_kib, _ = write[key]
        traffic = (f_kib * fs + w_kib * ws) * 1024
        rows.append(dict(workload=key, dispatches=n, fetch_kib=f_kib, write_kib=w_kib,
                         traffic=traffic, alg_bytes=alg[key], ratio=traffic / alg[key]))
    return rows, fs, ws


def format_trace(rows) -> str:
    out = [f"{'workload':<18}{'calls':>7}{'avg_ns':>11}{'min_ns':>9}{'max_ns':>9}{'alg_bytes':>12}"
           f"{'GB/s':>8}{'peak':>6}{'of_peak':>8}  kernel"]
    for r in rows:
        out.append(f"{r['workload']:<18}{r['calls']:>7}{r['avg_ns']:>11.0f}{r['min_ns']:>9.0f}"
                   f"{r['max_ns']:>9.0f}{r['alg_bytes']:>12}{r['gbps']:>8.0f}{r['peak']:>6}"
                   f"{r['of_peak']:>8.3f}  {r['kernel'][:100]}")
    return "\n".join(out) + "\n"


def format_traffic(rows, fs, ws, machine_lines: bool) -> str:
    out = [f"FETCH_SIZE reads {COPY_KIB_EACH_WAY / fs:,.1f} KiB per 4 GiB copy -> fetch scale "
           f"{fs:.4f}",
           f"WRITE_SIZE reads {COPY_KIB_EACH_WAY / ws:,.1f} KiB per 4 GiB copy -> write scale "
           f"{ws:.5f}",
           "traffic = (FETCH_SIZE * fetch scale + WRITE_SIZE * write scale) * 1024 bytes", "",
           f"{'workload':<18}{'dispatches':>11}{'FETCH_KiB':>12}{'WRITE_KiB':>12}{'traffic_B':>13}"
           f"{'alg_B':>13}{'ratio':>8}"]
    for r in rows:
        out.append(f"{r['workload']:<18}{r['dispatches']:>11}{r['fetch_kib']:>12.1f}"
                   f"{r['write_kib']:>12.1f}{r['traffic']:>13.0f}{r['alg_bytes']:>13}"
                   f"{r['ratio']:>8.4f}")
    if machine_lines:
        out += ["", "Machine-readable (bench.py reads these lines):"]
        out += [f"TRAFFIC {r['workload']} bytes_per_launch={r['traffic']:.0f} "
                f"fetch_kib={r['fetch_kib']:.1f} write_kib={r['write_kib']:.1f}"
                for r in rows if r["workload"] not in YARDSTICKS]
    return "\n".join(out) + "\n"


PRESETS = {
    "configs": dict(
        kernels=CONFIG_KERNELS, alg=config_bytes, machine=True,
        files=("row_kernels_all_configs_trace.txt", "row_kernels_all_configs_hbm_traffic.txt"),
        what="every measured workload (C1-C5, bench.py --all)",
        trace_cmd="python3 -u bench.py --all --no-cpu --steps 50",
        pmc_cmd="python3 -u bench.py --all --no-cpu --steps 50",
        source_note=("Trace calls include the single-launch timing, the 0.5 s warm-up, the warm-up\n"
                     "launches and the 50 timed launches of bench.py (the timed region alone is in\n"
                     "the *_timed_trace.txt summaries); the counters are averaged over the last 50\n"
                     "dispatches of each workload's kernel (--tail 50), which are bench.py's timed\n"
                     "launches.  Every input cycles through >= 2 GiB of HBM copies.")),
    "reference": dict(
        kernels=REFERENCE_KERNELS, alg=reference_bytes, machine=False,
        files=("reference_shapes_kernels_trace.txt", "reference_shapes_hbm_traffic.txt"),
        what="the family at the reference's large shapes (AKO4ALL/prepare_kernel.py KERNEL_CONFIGS)",
        trace_cmd="python3 -u -m dslperfgap_amd.viperbench.cliff_roofline --out RUN/cliff_traced.csv",
        pmc_cmd=("python3 -u -m dslperfgap_amd.viperbench.cliff_roofline --reps 10 --warmup 3 "
                 "--out RUN/cliff_COUNTER.csv"),
        source_note=("65 calls per kernel reuse one input set (the reference protocol); the rest\n"
                     "cycle through >= 2 GiB of HBM copies, so the averages are HBM-bound launches.")),
}


def _dir_prefix(path, suffix: str) -> tuple[str, str]:
    """(output directory, -o prefix) of a rocprofv3 csv file named <prefix><suffix>."""
    p = Path(path)
    name = p.name
    return str(p.parent), name[:-len(suffix)] if name.endswith(suffix) else name


def render(preset: str, trace, fetch, write, tail: int = 0) -> tuple[str, str]:
    """The trace summary and the traffic summary, headed by the commands that
    wrote the input files (directories and prefixes taken from their paths)."""
    p = PRESETS[preset]
    kernels, alg = p["kernels"], p["alg"]()
    order = [k for k, _ in kernels]
    stats = read_stats(trace, kernels)
    fetched, written = read_counter(fetch, kernels, tail), read_counter(write, kernels, tail)
    # a renamed kernel template must not drop a workload from the summaries
    # (bench.py reads the traffic lines)
    missing = [k for k in order if k != READ and
               (k not in stats or k not in fetched or k not in written)]
    if missing:
        raise ValueError(f"{preset}: no kernel in the rocprofv3 files matched {missing}; "
                         "update the symbol patterns")
    tr = trace_table(stats, alg, order)
    tdir, tpre = _dir_prefix(trace, "_kernel_stats.csv")
    run_dir = str(Path(tdir).parent)
    cmd = p["trace_cmd"].replace("RUN", run_dir)
    head = (f"rocprofv3 kernel trace -- {p['what']} (MI355X, gfx950)\n\n"
            f"Command (from the repository root, after `cd /tmp && export TMPDIR=/tmp`):\n"
            f"  rocprofv3 --kernel-trace --stats --output-format csv -d {tdir} -o {tpre} -- \\\n"
            f"      {cmd}\n"
            f"Summary: python -m dslperfgap_amd.viperbench.rocprof_summary {preset} ...\n\n"
            f"{p['source_note']}\n"
            f"achieved = algorithmic bytes / AverageNs (ns); of_peak = achieved / the rate of the\n"
            f"kernel's measured yardstick in the same run (peak: copy = the 4 GiB stream copy,\n"
            f"read + write; read = the 4 GiB streaming read, for the kernels that write almost\n"
            f"nothing).\n\n")
    trace_txt = head + format_trace(tr)
    rows, fs, ws = traffic_table(fetched, written, alg, order)
    pmc = []
    for c, path in (("FETCH_SIZE", fetch), ("WRITE_SIZE", write)):
        d, pre = _dir_prefix(path, "_counter_collection.csv")
        pmc.append(f"  timeout -s KILL 400 rocprofv3 --pmc {c} --output-format csv -d {d} -o {pre} -- \\\n"
                   f"      {p['pmc_cmd'].replace('RUN', run_dir).replace('COUNTER', c)}")
    pmc = "\n".join(pmc)
    head = (f"rocprofv3 HBM traffic counters -- {p['what']} (MI355X, gfx950)\n\n"
            f"Commands (from the repository root, after `cd /tmp && export TMPDIR=/tmp`), one\n"
            f"counter per run:\n{pmc}\n"
            f"Summary: python -m dslperfgap_amd.viperbench.rocprof_summary {preset} ...\n\n"
            f"Counter values are KiB per dispatch, averaged over the dispatches named above,\n"
            f"scaled by what each counter reads for the 4 GiB copy kernel of the same runs.\n\n")
    return trace_txt, head + format_traffic(rows, fs, ws, p["machine"])


# Instruction counters of the "pipes" summary, in table order.  SQ_INSTS_* and
# SQ_WAVES are totals per dispatch over every shader engine of the 8 XCDs.
PIPE_COUNTERS = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_SALU",
                 "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR", "VALUBusy")
PIPES_FILE = "row_kernels_all_configs_instruction_counters.txt"
SIMDS = 256 * 4                     # MI355X: 256 CUs x 4 SIMDs
PEAK_CLOCK_HZ = 2.4e9               # MI355X peak engine clock
VALU_CYCLES = 4                     # a wave64 VALU instruction on a 16-lane SIMD


def config_elements() -> dict:
    """Input elements per launch of each config (rows x columns of the row
    input; 4-byte words for the 4 GiB yardsticks)."""
    shapes = {"C1_layer_norm": (4096, 1024), "C2_rms_norm": (8192, 4096),
              "C3_softmax": (16384, 4096), "C3_log_softmax": (16384, 4096),
              "C3_logsumexp": (16384, 4096), "C4_cross_entropy": (8192, 32000),
              "C4_cross_entropy_bwd": (8192, 32000), "C5_layer_norm": (2048, 20480)}
    out = {k: r * c for k, (r, c) in shapes.items()}
    out[COPY] = out[READ] = (4 << 30) // 4
    return out


def read_counters(paths, kernels, tail: int = 0) -> dict:
    """{workload: {counter: mean value per dispatch}} from one or more
    counter_collection.csv files (a counter found in several files is taken
    from the first); `tail` as in read_counter."""
    out: dict = collections.defaultdict(dict)
    for path in paths:
        acc = collections.defaultdict(lambda: collections.defaultdict(float))
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                key = classify(r["Kernel_Name"], kernels)
                if key:
                    acc[(key, r["Counter_Name"])][int(r["Dispatch_Id"])] += float(r["Counter_Value"])
        for (key, counter), per in acc.items():
            if counter in out[key]:
                continue
            ids = sorted(per)
            if tail and key != COPY:
                ids = ids[-tail:]
            out[key][counter] = sum(per[i] for i in ids) / len(ids)
    return dict(out)


def pipes_table(counters: dict, stats: dict, elements: dict, order) -> list[dict]:
    rows = []
    for key in order:
        c = counters.get(key)
        if not c or "SQ_WAVES" not in c or key not in stats:
            continue
        waves = c["SQ_WAVES"]
        per_wave = {n: c[n] / waves for n in PIPE_COUNTERS[1:6] if n in c}
        valu = c.get("SQ_INSTS_VALU", float("nan"))
        floor_ns = valu * VALU_CYCLES / SIMDS / PEAK_CLOCK_HZ * 1e9
        avg = stats[key][2]
        rows.append(dict(workload=key, waves=waves, per_wave=per_wave,
                         valu_per_64=valu / (elements[key] / 64), avg_ns=avg,
                         valu_floor_ns=floor_ns, floor_share=floor_ns / avg,
                         valu_busy=c.get("VALUBusy", float("nan"))))
    return rows


def reference_elements() -> dict:
    """Input elements per launch of each kernel at the reference's large shape
    (cliff_roofline.py's ENTRIES; 4-byte words for the 4 GiB yardsticks)."""
    sq, wide = 8192 * 8192, 8192 * 32768
    return {"layer_norm": sq, "rms_norm": sq, "softmax": 4096 * 32768,
            "log_softmax": 4096 * 32768, "logsumexp": 8192 * 16384,
            "cross_entropy": 4096 * 32768, "argmax": wide, "max_reduction": wide,
            "mean_reduction": wide, COPY: (4 << 30) // 4, READ: (4 << 30) // 4}


PIPE_TARGETS = {
    "configs": dict(kernels=lambda: CONFIG_KERNELS, elements=lambda: config_elements(),
                    cmd=lambda: PRESETS["configs"]["pmc_cmd"], file=PIPES_FILE,
                    what="every measured workload (C1-C5, bench.py --all)",
                    tail_note="bench.py's timed launches"),
    "reference": dict(kernels=lambda: REFERENCE_KERNELS, elements=lambda: reference_elements(),
                      cmd=lambda: ("python3 -u -m dslperfgap_amd.viperbench.cliff_roofline "
                                   "--out RUN/cliff_pipes.csv"),
                      file="reference_shapes_instruction_counters.txt",
                      what="the family at the reference's large shapes (cliff_roofline.py)",
                      tail_note="the HBM-cycled launches cliff_roofline.py times last"),
}


def render_pipes(trace, pmcs, tail: int = 0, bench_lines=None, of: str = "configs") -> str:
    tgt = PIPE_TARGETS[of]
    kernels = tgt["kernels"]()
    order = [k for k, _ in kernels]
    stats = read_stats(trace, kernels)
    counters = read_counters(pmcs, kernels, tail)
    missing = [k for k in order if k != READ and (k not in stats or k not in counters)]
    if missing:
        raise ValueError(f"pipes: no kernel in the rocprofv3 files matched {missing}; "
                         "update the symbol patterns")
    rows = pipes_table(counters, stats, tgt["elements"](), order)
    tdir, tpre = _dir_prefix(trace, "_kernel_stats.csv")
    cmd = tgt["cmd"]().replace("RUN", str(Path(tdir).parent))
    runs = []
    for path in pmcs:
        d, pre = _dir_prefix(path, "_counter_collection.csv")
        with open(path, newline="") as f:
            names = sorted({r["Counter_Name"] for r in csv.DictReader(f)})
        runs.append(f"  timeout -s KILL 400 rocprofv3 --pmc {' '.join(names)} \\\n"
                    f"      --output-format csv -d {d} -o {pre} -- {cmd}")
    head = [
        f"rocprofv3 instruction counters -- {tgt['what']} (MI355X, gfx950)", "",
        "Commands (from the repository root, after `cd /tmp && export TMPDIR=/tmp`), one run",
        "per counter group, and the kernel trace the durations come from:", *runs,
        f"  rocprofv3 --kernel-trace --stats --output-format csv -d {tdir} -o {tpre} -- {cmd}",
        "Summary: python -m dslperfgap_amd.viperbench.rocprof_summary pipes \\",
        f"      --of {of} --trace <stats csv> --pmc <counter csv> ... --tail {tail}"
        + (" --bench-lines <bench.py lines>" if of == "configs" else ""),
        "",
        "Counters are totals per dispatch (every shader engine of the 8 XCDs), averaged over",
        f"the last {tail} dispatches of each workload's kernel ({tgt['tail_note']}; the",
        "yardsticks over all of theirs); per-wave figures divide by SQ_WAVES.",
        "VALU/64el = VALU instructions per 64 input elements (one wave64 instruction per",
        "element would be 1.0).  VALU floor = SQ_INSTS_VALU x 4 cycles / 1024 SIMDs at the",
        "2.4 GHz peak clock: the time the SIMDs need just to issue the VALU instructions",
        "(transcendentals and dependency stalls take longer), against the traced average",
        "duration avg_ns.  VALUBusy = rocprofv3's derived counter (100 x SQ_ACTIVE_INST_VALU",
        "/ CU count / GRBM_GUI_ACTIVE), the share of the dispatch's cycles the SIMDs spent",
        "on VALU work.", ""]
    if bench_lines:
        import json

        hashes = sorted({json.loads(ln).get("lib_srchash", "") for ln in
                         Path(bench_lines).read_text().splitlines() if ln.strip().startswith("{")}
                        - {""})
        if hashes:
            head.insert(1, f"Library source hash (libvbhip.srchash, csrc/ + include/): "
                           f"{', '.join(hashes)}")
    hdr = (f"{'workload':<21}{'waves':>9}{'VALU/wave':>10}{'trans/wave':>11}{'SALU/wave':>10}"
           f"{'VMEMrd/w':>9}{'VMEMwr/w':>9}{'VALU/64el':>10}{'avg_ns':>10}{'VALUfloor':>10}"
           f"{'floor%':>7}{'VALUBusy%':>10}")
    lines = [hdr]
    for r in rows:
        pw = r["per_wave"]
        lines.append(
            f"{r['workload']:<21}{r['waves']:>9.0f}{pw.get('SQ_INSTS_VALU', float('nan')):>10.1f}"
            f"{pw.get('SQ_INSTS_VALU_TRANS_F32', float('nan')):>11.1f}"
            f"{pw.get('SQ_INSTS_SALU', float('nan')):>10.1f}"
            f"{pw.get('SQ_INSTS_VMEM_RD', float('nan')):>9.1f}"
            f"{pw.get('SQ_INSTS_VMEM_WR', float('nan')):>9.1f}{r['valu_per_64']:>10.2f}"
            f"{r['avg_ns']:>10.0f}{r['valu_floor_ns']:>10.0f}{100 * r['floor_share']:>7.1f}"
            f"{r['valu_busy']:>10.1f}")
    return "\n".join(head + lines) + "\n"


TIMED_PREFIX = "vbh-timed:"


def read_dispatches(path) -> list[dict]:
    """Kernel dispatches of a ``<prefix>_kernel_trace.csv``: name, start, end (ns)."""
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            out.append(dict(name=r["Kernel_Name"], start=int(r["Start_Timestamp"]),
                            end=int(r["End_Timestamp"]), dispatch=int(r["Dispatch_Id"])))
    return out


def read_ranges(path) -> list[dict]:
    """bench.py's timed roctx ranges from a ``<prefix>_marker_api_trace.csv``:
    the rows whose function (the range's message) starts with ``vbh-timed:``."""
    out = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            msg = r.get("Function") or r.get("Message") or ""
            if msg.startswith(TIMED_PREFIX):
                _, key, steps = msg.split(":")
                out.append(dict(workload=key, steps=int(steps), start=int(r["Start_Timestamp"]),
                                end=int(r["End_Timestamp"])))
    return out


def alg_bytes_of(key: str) -> int:
    """Algorithmic bytes per launch of a workload key, or of ``copy@N`` (the
    stream copy moving N bytes per launch, read + write) or ``read@N`` (the
    streaming read of N bytes per launch)."""
    if key.startswith(YARDSTICK_KINDS):
        return int(key.split("@", 1)[1])
    return WORKLOADS[key].bytes_per_launch


# bench.py's yardstick lines: key prefix -> command-line option
YARDSTICK_KINDS = ("copy@", "read@", "runtime_copy@")


def timed_row(dispatches: list[dict], rng: dict, alg_bytes: int) -> dict:
    """Statistics of the dominant kernel (most device time) among the dispatches
    that ran entirely inside the timed range."""
    inside = [d for d in dispatches if d["start"] >= rng["start"] and d["end"] <= rng["end"]]
    if not inside:
        raise ValueError(f"no kernel dispatch inside the timed range of {rng['workload']}")
    by_name = collections.defaultdict(list)
    for d in inside:
        by_name[d["name"]].append(d)
    name, ds = max(by_name.items(), key=lambda kv: sum(d["end"] - d["start"] for d in kv[1]))
    ds.sort(key=lambda d: d["start"])
    dur = sorted(d["end"] - d["start"] for d in ds)
    n = len(dur)
    avg = sum(dur) / n
    span = ds[-1]["end"] - ds[0]["start"]
    return dict(workload=rng["workload"], steps=rng["steps"], kernel=name, calls=n,
                others=len(inside) - n, avg_ns=avg, min_ns=dur[0], max_ns=dur[-1],
                median_ns=dur[n // 2], period_ns=span / n, alg_bytes=alg_bytes,
                gbps=alg_bytes / avg, gbps_period=alg_bytes / (span / n))


def kernel_base(kernel: str) -> str:
    """Base name of a kernel symbol: ``ce_fwd_rows`` for
    ``void vbh::(anonymous namespace)::ce_fwd_rows<float, ...>(...)`` and for
    the Itanium-mangled ``_ZN3vbh12_GLOBAL__N_111ce_fwd_rowsI...``."""
    if kernel.startswith("_ZN"):
        i, last = 3, None
        while i < len(kernel) and kernel[i].isdigit():
            j = i
            while kernel[j].isdigit():
                j += 1
            n = int(kernel[i:j])
            last, i = kernel[j:j + n], j + n
        return last or "kernel"
    head = kernel.replace("(anonymous namespace)", "").split("(")[0].split("<")[0]
    return head.split("::")[-1].split()[-1] if head.strip() else "kernel"


def timed_file(workload: str, kernel: str) -> str:
    """``<kernel>_<workload>_timed_trace.txt`` (kernel = the symbol's base name)."""
    return f"{kernel_base(kernel)}_{workload.replace('@', '_')}_timed_trace.txt"


def render_timed(kernel_trace, markers, bench_lines) -> tuple[str, dict]:
    """Summary of the kernel dispatches inside each timed range of
    ``bench.py`` (one range per workload), next to bench.py's own lines from
    the same run.  Returns the combined text and {workload: (file name, text)}."""
    import json

    dispatches = read_dispatches(kernel_trace)
    ranges = read_ranges(markers)
    if not ranges:
        raise ValueError(f"{markers}: no {TIMED_PREFIX} range (was bench.py run under "
                         "rocprofv3 --marker-trace?)")
    lines = {}
    for ln in Path(bench_lines).read_text().splitlines():
        ln = ln.strip()
        if ln.startswith("{"):
            d = json.loads(ln)
            lines[d["config"]["workload"]] = d
    tdir, tpre = _dir_prefix(kernel_trace, "_kernel_trace.csv")
    rows = [timed_row(dispatches, r, alg_bytes_of(r["workload"])) for r in ranges]
    keys = [r["workload"] for r in rows]
    sizes = {kind: [k.split("@", 1)[1] for k in keys if k.startswith(kind + "@")]
             for kind in ("copy", "read", "runtime_copy")}
    yard = " ".join(f"--{kind.replace('_', '-')}-at " + " ".join(v)
                    for kind, v in sizes.items() if v)
    work = [k for k in keys if not k.startswith(YARDSTICK_KINDS)]
    if len(work) > 1:
        args = "--all"
    elif work:
        args = "" if work == ["C4_cross_entropy"] and not yard else f"--workload {work[0]}"
    else:
        args = ""
    args = f"{args} {yard}".strip()
    graphed = any("graph" in lines.get(k, {}).get("timing", "") for k in work)
    steps = rows[0]["steps"]
    step_arg = "" if steps == 1000 else f" --steps {steps}"
    extra = (" --graph" if graphed else "") + (" --no-per-config" if not args or
                                                args == yard else "")
    cmd = f"python3 -u bench.py {args}{step_arg} --no-cpu{extra}".replace("  ", " ")
    head = [f"rocprofv3 kernel trace of bench.py's timed regions (MI355X, gfx950)", "",
            "Command (from the repository root, after `cd /tmp && export TMPDIR=/tmp`):",
            f"  rocprofv3 --kernel-trace --marker-trace --output-format csv -d {tdir} -o {tpre} -- \\",
            f"      {cmd} > BENCH_LINES",
            f"Summary: python -m dslperfgap_amd.viperbench.rocprof_summary timed \\",
            f"      --kernel-trace {kernel_trace} --markers {markers} --bench-lines BENCH_LINES", "",
            "Only dispatches that ran entirely inside bench.py's roctx range",
            "vbh-timed:<workload>:<steps> are counted: the timed launches, nothing of the",
            "warm-up.  avg_ns = mean kernel duration; period_ns = (end of the last - start of",
            "the first) / calls, the per-launch time the device events of bench.py measure",
            "(kernel + gap to the next launch).  GB/s = algorithmic bytes / avg_ns;",
            "GB/s_period = algorithmic bytes / period_ns.", ""]
    table = [f"{'workload':<21}{'calls':>6}{'avg_ns':>10}{'med_ns':>10}{'min_ns':>9}{'max_ns':>9}"
             f"{'period_ns':>11}{'GB/s':>7}{'GB/s_period':>12}{'bench_us':>10}{'period/bench':>13}"]
    for r in rows:
        b = lines.get(r["workload"], {})
        lat = b.get("latency_us")
        r["bench_latency_us"] = lat
        r["agree"] = (r["period_ns"] / 1e3) / lat if lat else float("nan")
        table.append(f"{r['workload']:<21}{r['calls']:>6}{r['avg_ns']:>10.0f}{r['median_ns']:>10.0f}"
                     f"{r['min_ns']:>9.0f}{r['max_ns']:>9.0f}{r['period_ns']:>11.0f}"
                     f"{r['gbps']:>7.0f}{r['gbps_period']:>12.0f}"
                     f"{lat if lat is not None else float('nan'):>10.3f}{r['agree']:>13.4f}")
    kernels = ["", "Kernels:"] + [f"  {r['workload']}: {r['kernel'][:150]}"
                                  + (f"  (+{r['others']} other dispatches in the range)"
                                     if r["others"] else "")
                                  + (f"  (range named {r['steps']} steps, {r['calls']} dispatches)"
                                     if r["calls"] != r["steps"] else "") for r in rows]
    hashes = sorted({b.get("lib_srchash") for b in lines.values() if b.get("lib_srchash")})
    if hashes:
        head.insert(1, f"Library source hash (libvbhip.srchash, csrc/ + include/): "
                       f"{', '.join(hashes)}")
    bench = ["", "bench.py lines of the traced run (value GB/s, latency_us, roofline.frac):"]
    for k in keys:
        b = lines.get(k)
        if b:
            of = (f", of measured {b['measured_peak_kind']} peak {b['frac_of_measured_peak']}"
                  if "measured_peak_kind" in b else "")
            bench.append(f"  {k}: {b['value']} GB/s, {b['latency_us']} us, "
                         f"frac {b['roofline']['frac']}{of}")
    combined = "\n".join(head + table + kernels + bench) + "\n"
    per = {}
    for r in rows:
        i = keys.index(r["workload"])
        one = "\n".join(head + [table[0], table[1 + i], "", "Kernel:", f"  {r['kernel']}"]
                        + bench[:2] + [x for x in bench[2:]
                                       if x.startswith(f"  {r['workload']}:")]) + "\n"
        per[r["workload"]] = (timed_file(r["workload"], r["kernel"]), one)
    return combined, per


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("preset", choices=sorted(PRESETS) + ["timed", "pipes"])
    ap.add_argument("--trace", help="<prefix>_kernel_stats.csv")
    ap.add_argument("--kernel-trace", help="timed: <prefix>_kernel_trace.csv")
    ap.add_argument("--markers", help="timed: <prefix>_marker_api_trace.csv")
    ap.add_argument("--combined-name", default=None,
                    help="timed: also write the table of every range under this file name")
    ap.add_argument("--fetch", help="FETCH_SIZE <prefix>_counter_collection.csv")
    ap.add_argument("--write", help="WRITE_SIZE <prefix>_counter_collection.csv")
    ap.add_argument("--pmc", action="append", default=[],
                    help="pipes: a <prefix>_counter_collection.csv of instruction counters "
                         "(repeatable)")
    ap.add_argument("--bench-lines", help="timed, pipes: the JSON lines bench.py printed in the "
                                          "run")
    ap.add_argument("--tail", type=int, default=0,
                    help="counters: only the last TAIL dispatches of each workload's kernel "
                         "(bench.py's timed launches are each workload's last ones)")
    ap.add_argument("--of", choices=sorted(PIPE_TARGETS), default="configs",
                    help="pipes: the configs (bench.py --all) or the reference's large shapes")
    ap.add_argument("--out-dir", default=None, help="write the summaries here (else print)")
    args = ap.parse_args(argv)
    if args.preset == "timed":
        if not (args.kernel_trace and args.markers and args.bench_lines):
            ap.error("timed needs --kernel-trace, --markers and --bench-lines")
        combined, per = render_timed(args.kernel_trace, args.markers, args.bench_lines)
        if args.out_dir:
            # one range: a file named for its kernel and workload; several: the
            # combined table under --combined-name
            if len(per) == 1 or not args.combined_name:
                for name, txt in per.values():
                    Path(args.out_dir, name).write_text(txt)
            if args.combined_name:
                Path(args.out_dir, args.combined_name).write_text(combined)
        else:
            sys.stdout.write(combined)
        return 0
    if args.preset == "pipes":
        if not (args.trace and args.pmc):
            ap.error("pipes needs --trace and at least one --pmc")
        txt = render_pipes(args.trace, args.pmc, tail=args.tail, bench_lines=args.bench_lines,
                           of=args.of)
        if args.out_dir:
            Path(args.out_dir, PIPE_TARGETS[args.of]["file"]).write_text(txt)
        else:
            sys.stdout.write(txt)
        return 0
    if not (args.trace and args.fetch and args.write):
        ap.error(f"{args.preset} needs --trace, --fetch and --write")
    trace_txt, traffic_txt = render(args.preset, args.trace, args.fetch, args.write,
                                    tail=args.tail)
    if args.out_dir:
        names = PRESETS[args.preset]["files"]
        Path(args.out_dir, names[0]).write_text(trace_txt)
        Path(args.out_dir, names[1]).write_text(traffic_txt)
    else:
        sys.stdout.write(trace_txt + "\n" + traffic_txt)
    return 0


if __name__ == "__main__":
    sys.exit(main())
