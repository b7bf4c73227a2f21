#!/usr/bin/env python
"""Benchmark of the draft-objective hot path on one MI355X.

Metric: draft slots/sec, forward + backward (CE + KL + accept_len forward, dl,
and dhidden when the LM head is fused), with the dominant kernel's roofline
fraction.  A "step" is one pass of the hot path over one batch of synthetic
input that is already resident in HBM.

    python bench.py [--steps K] [--warmup W] [--config c1|c2|c2x|c3|c4]

Prints ONE JSON line.  By default the headline is C2 (the configuration the metric is
quoted on) and C1, C3, C4 and C2X follow in the same process under "secondary".  One GPU only: ``--gpus N`` with N > 1 exits with a
message (the path is data-parallel over slots; the library has no collectives).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
FP8_PEAK_TFLOPS = 5000.0       # MI355X dense fp8 MFMA, TFLOP/s
WARMUP_MIN_S = 0.25            # untimed warmup: at least --warmup steps and at least this long
WARMUP_MAX_STEPS = 2000

METRIC = "draft slots/sec fwd+bwd CE+KL+accept @V=248k,d=5120; %MFMA & %HBM roof"


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default=None, choices=["c1", "c2", "c3", "c3s", "c4", "c2x"],
                   help="one workload alone; default: C2 (the headline), then C1, C3, C4 and C2X as secondary lines")
    p.add_argument("--no-secondary", action="store_true", help="default run: C2 only")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--markov-skew", type=float, default=0.0,
                   help="c2x: fraction of rows sharing one previous-token id (the W1 scatter's worst case)")
    p.add_argument("--cpu-rows", type=int, default=0, help="rows in the CPU-baseline sample (0: default)")
    p.add_argument("--pmc-driver", action="store_true",
                   help="short run for one rocprofv3 --pmc pass: a 1 GiB calibration kernel, then two steps")
    p.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="print the HBM-traffic summary of two --pmc-driver passes (FETCH_SIZE, WRITE_SIZE)")
    p.add_argument("--stats-from", metavar="DIR", help="print a summary of a rocprofv3 --stats csv run")
    p.add_argument("--mfma-from", metavar="DIR",
                   help="print the matrix-core summary of one --pmc-driver pass with the MFMA counters")
    p.add_argument("--memory-from", nargs="+", metavar="DIR",
                   help="print the L1/L2 read-pipeline summary of the --pmc-driver passes with MEMORY_PASSES")
    p.add_argument("--command", default="", help="command line recorded in a printed summary")
    return p.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# --------------------------------------------------------------------------- profiles

# library kernel symbol (demangled, as rocprofv3 prints it) -> the launch-site name the
# library's own timer (ns_profile_*) uses
KERNEL_NAMES = [
    (r"head_kernel<0,", "head_stats"),
    (r"head_kernel<1,", "head_emit"),
    (r"head_kernel<2,", "head_linear"),
    (r"dh_reduce_kernel", "dh_reduce"),
    (r"dh_kernel", "dh_gemm"),
    (r"stream_stats_kernel", "stream_stats"),
    (r"stream_group_kernel<[^,]+, [^,]+, true>", "stream_group"),
    (r"stream_group_kernel<[^,]+, [^,]+, false>", "stream_group_accept"),
    (r"group_clear_kernel", "group_clear"),
    # stream_emit_kernel<TZ, TU, TD, VEC, EMIT, ACCEPT>
    (r"stream_emit_kernel<[^,]+, [^,]+, [^,]+, (?:true|false), true", "stream_emit"),
    (r"stream_emit_kernel<[^,]+, [^,]+, [^,]+, (?:true|false), false", "stream_accept"),
    (r"lse_merge_kernel", "lse_merge"),
    (r"merge_kernel", "merge_rows"),
    (r"finalize_kernel", "finalize_metrics"),
    (r"row_parts_kernel", "row_parts"),
    (r"accept_rows_kernel", "accept_rows"),
    (r"sum_partials_kernel", "dprev_reduce"),
    (r"gather_rows_kernel", "markov_gather"),
    (r"dw2_kernel", "markov_dw2"),
    (r"markov_(?:sort_chunks|merge)_kernel", "markov_sort"),
    (r"markov_(?:pieces|runs)_kernel", "markov_scatter"),
    (r"rms_fwd_kernel", "rms_norm_fwd"),
    (r"rms_bwd_kernel", "rms_norm_bwd"),
    (r"rms_wgrad_kernel", "rms_norm_wgrad"),
    (r"pooled_tail_kernel", "pooled_tail"),
    (r"scale_kernel", "scale_gradient"),
    (r"fp8_quant_kernel", "fp8_quant"),
    (r"fp8_head_kernel", "fp8_head_gemm"),
    (r"copy_rows_kernel", "copy_rows"),
    (r"prepare_kernel", "prepare_slots"),
]
# profiles/<prefix>_traffic.md and <prefix>_kernel_stats.md: named for the kernels and workload
PROFILE_PREFIX = {"c1": "stream_c1", "c2": "lmhead_c2", "c3": "lmhead_c3", "c3s": "lmhead_c3s",
                  "c4": "fp8_lmhead_c4", "c2x": "head_ext_c2x"}
CALIBRATION_BYTES = 1 << 30   # the --pmc-driver calibration (fp32 negation): reads and writes 1 GiB


def timer_name(kernel: str):
    import re

    if "ns::" not in kernel:
        return None
    for pat, name in KERNEL_NAMES:
        if re.search(pat, kernel):
            return name
    return None


def _csv_rows(directory: str, suffix: str):
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {directory}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _launches(counters, durations):
    """Per-launch records from one pass's per-dispatch ones ({dispatch id: (kernel name,
    {counter: value})} and {dispatch id: ns}).  A run of consecutive dispatches of one library
    kernel is one launch: the library issues a long GEMM as one launch per round of
    workgroups inside one timer scope (the dh GEMM past five rounds).  Its counters and
    durations are summed.  Returns [(timer name, {counter: sum}, ns or None, dispatches)] for
    the library kernels."""
    out, prev = [], None
    for d in sorted(counters):
        kname, vals = counters[d]
        name = timer_name(kname)
        dur = durations.get(d)
        if name is not None and name == prev:
            _, acc, ns, k = out[-1]
            for c, v in vals.items():
                acc[c] = acc.get(c, 0.0) + v
            out[-1] = (name, acc, None if ns is None or dur is None else ns + dur, k + 1)
        elif name is not None:
            out.append((name, dict(vals), dur, 1))
        prev = name
    return out


def _counter_per_kernel(directory: str, counter: str):
    """Median per-launch value (KiB) of `counter` for each library kernel, plus the
    calibration kernel's value."""
    import statistics

    counters, calib = {}, []
    seen_library = False   # the calibration kernel follows the driver's first step
    rows = [r for r in _csv_rows(directory, "counter_collection.csv") if r["Counter_Name"] == counter]
    for r in sorted(rows, key=lambda r: int(r["Dispatch_Id"])):
        counters[int(r["Dispatch_Id"])] = (r["Kernel_Name"], {counter: float(r["Counter_Value"])})
        if timer_name(r["Kernel_Name"]):
            seen_library = True
        elif seen_library and "neg" in r["Kernel_Name"]:
            calib.append(float(r["Counter_Value"]))
    if not calib:
        raise SystemExit(f"no calibration dispatch (torch.neg) in {directory}")
    per = {}
    for name, vals, _, _ in _launches(counters, {}):
        per.setdefault(name, []).append(vals[counter])
    return {k: statistics.median(v) for k, v in per.items()}, max(calib)


def traffic_summary(fetch_dir: str, write_dir: str, config: str, command: str) -> str:
    """Markdown: per-kernel HBM bytes per launch from FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled so that the calibration kernel reads (writes) exactly 1 GiB."""
    fetch, fcal = _counter_per_kernel(fetch_dir, "FETCH_SIZE")
    write, wcal = _counter_per_kernel(write_dir, "WRITE_SIZE")
    ff = CALIBRATION_BYTES / (fcal * 1024.0)
    wf = CALIBRATION_BYTES / (wcal * 1024.0)
    out = [f"# HBM traffic per launch: {config.upper()} kernels (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
           "Commands (from the repository root on the MI355X box):", "", "```", command.strip(), "```", "",
           "Each counter pass runs `bench.py --pmc-driver`: one step, a torch fp32 negation of 1 GiB into another "
           "1 GiB (the calibration kernel), then two steps. The calibration kernel reads "
           f"{fcal:.0f} KiB and writes {wcal:.0f} KiB by the counters, so FETCH_SIZE is scaled by "
           f"{ff:.4f} and WRITE_SIZE by {wf:.4f}. Values are per-launch medians (a launch issued as one dispatch "
           "per round of workgroups sums its dispatches); FETCH_SIZE counts L2 fills "
           "from the fabric, which include Infinity Cache (MALL) hits.", "",
           "| kernel | fetch GB | write GB | traffic GB |", "|---|---:|---:|---:|"]
    machine = []
    for name in sorted(set(fetch) | set(write)):
        fb = fetch.get(name, 0.0) * 1024.0 * ff
        wb = write.get(name, 0.0) * 1024.0 * wf
        out.append(f"| `{name}` | {fb / 1e9:.3f} | {wb / 1e9:.3f} | {(fb + wb) / 1e9:.3f} |")
        machine.append(f"traffic {name} fetch_bytes={fb:.0f} write_bytes={wb:.0f}")
    out += ["", "Machine-readable (read by bench.py for `roofline.traffic`):", "", "```"] + machine + ["```", ""]
    return "\n".join(out)


def stats_summary(directory: str, config: str, command: str) -> str:
    rows = _csv_rows(directory, "kernel_stats.csv")
    # launches per kernel from the same run's kernel trace (a launch issued as one dispatch per
    # round of workgroups counts once); the column appears only when they differ from calls
    launches = {}
    try:
        trace = {int(r["Dispatch_Id"]): (r["Kernel_Name"], {}) for r in _csv_rows(directory, "kernel_trace.csv")}
    except SystemExit:
        trace = {}
    for name, _, _, _ in _launches(trace, {}):
        launches[name] = launches.get(name, 0) + 1
    split = any(launches.get(timer_name(r["Name"]), int(r["Calls"])) != int(r["Calls"])
                for r in rows if timer_name(r["Name"]))
    head = "| kernel | timer name | calls | total ms | average ms | % of GPU time |"
    rule = "|---|---|---:|---:|---:|---:|"
    if split:
        head = "| kernel | timer name | calls | launches | total ms | average ms per call | average ms per launch | % of GPU time |"
        rule = "|---|---|---:|---:|---:|---:|---:|---:|"
    out = [f"# rocprofv3 kernel stats: {config.upper()}", "", "Command (from the repository root on the MI355X box):",
           "", "```", command.strip(), "```", ""]
    if split:
        out += ["A launch is one timer scope of the library: the dh GEMM past five rounds of workgroups is "
                "issued as one dispatch per round, so its calls are several per launch.", ""]
    out += [head, rule]
    other = 0.0
    for r in rows:
        name = timer_name(r["Name"])
        if not name:
            other += float(r["Percentage"])
            continue
        short = r["Name"].replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")
        if len(short) > 90:
            short = short[:87] + "..."
        total = float(r["TotalDurationNs"]) / 1e6
        if split:
            n_l = launches.get(name, int(r["Calls"]))
            out.append(f"| `{short}` | {name} | {r['Calls']} | {n_l} | {total:.3f} | "
                       f"{float(r['AverageNs']) / 1e6:.4f} | {total / max(n_l, 1):.4f} | {float(r['Percentage']):.1f} |")
        else:
            out.append(f"| `{short}` | {name} | {r['Calls']} | {total:.3f} | "
                       f"{float(r['AverageNs']) / 1e6:.4f} | {float(r['Percentage']):.1f} |")
    cols = "| | | | | | |" if split else "| | | | |"
    out.append(f"| (torch input generation and copies, outside the timed steps) {cols} {other:.1f} |")
    out.append("")
    return "\n".join(out)


def committed_traffic(config: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed traffic summary, or None."""
    import re

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{PROFILE_PREFIX[config]}_traffic.md")
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(rf"^traffic {re.escape(kernel)} fetch_bytes=(\d+) write_bytes=(\d+)$", text, re.M)
    if not m:
        return None
    return int(m.group(1)) + int(m.group(2)), os.path.relpath(path, os.path.dirname(os.path.abspath(__file__)))


MFMA_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F8", "SQ_VALU_MFMA_BUSY_CYCLES",
                 "GRBM_GUI_ACTIVE")
SIMDS = 1024                        # MI355X: 256 CUs x 4 SIMDs
FLOP_PER_CLK_SIMD = {"bf16": 1024.0, "fp8": 2048.0}   # dense MFMA: 2.5 (5.0) PFLOP/s at 2.4 GHz


def _per_dispatch(directory: str):
    """{dispatch id: (kernel name, {counter: value})} of one --pmc pass, plus
    {dispatch id: duration ns} from the same run's kernel trace."""
    counters = {}
    for r in _csv_rows(directory, "counter_collection.csv"):
        d = int(r["Dispatch_Id"])
        counters.setdefault(d, (r["Kernel_Name"], {}))[1][r["Counter_Name"]] = float(r["Counter_Value"])
    durations = {}
    for r in _csv_rows(directory, "kernel_trace.csv"):
        durations[int(r["Dispatch_Id"])] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    return counters, durations


def mfma_summary(directory: str, config: str, command: str) -> str:
    """Markdown: the matrix cores of each library GEMM kernel from one rocprofv3 pass with
    MFMA_COUNTERS and --kernel-trace (per-launch medians):
    * executed FLOP = MOPS x 512 (bf16 or fp8), to check against the algorithmic count;
    * clock = GRBM_GUI_ACTIVE / duration, where GRBM_GUI_ACTIVE is summed over the 8 XCDs
      (so it is divided by 8);
    * mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (cycles x 1024 SIMDs);
    * per_clock = executed FLOP / (cycles x 1024 SIMDs x dense FLOP per SIMD per clock): the
      fraction of the matrix cores' peak at the clock the chip actually ran."""
    import statistics

    counters, durations = _per_dispatch(directory)
    per = {}
    for name, vals, ns, _ in _launches(counters, durations):
        if ns is None or not all(c in vals for c in MFMA_COUNTERS):
            continue
        bf, f8 = vals["SQ_INSTS_VALU_MFMA_MOPS_BF16"], vals["SQ_INSTS_VALU_MFMA_MOPS_F8"]
        if bf + f8 == 0:
            continue
        dtype = "fp8" if f8 > bf else "bf16"
        flop = 512.0 * (f8 if dtype == "fp8" else bf)
        dur = ns * 1e-9
        cycles = vals["GRBM_GUI_ACTIVE"] / 8.0
        per.setdefault(name, []).append(dict(
            dtype=dtype, flop=flop, ms=dur * 1e3, clock_GHz=cycles / dur / 1e9,
            mfma_busy=vals["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * SIMDS),
            per_clock=flop / (cycles * SIMDS * FLOP_PER_CLK_SIMD[dtype]),
            peak_frac=flop / dur / (2.5e15 if dtype == "bf16" else 5.0e15)))
    if not per:
        raise SystemExit(f"no library MFMA dispatches with {MFMA_COUNTERS} in {directory}")
    out = [f"# Matrix cores per GEMM kernel: {config.upper()} (rocprofv3 MFMA counters)", "",
           "Command (from the repository root on the MI355X box):", "", "```", command.strip(), "```", "",
           "One `bench.py --pmc-driver` pass (one step, a calibration copy, two steps) with "
           f"`--pmc {' '.join(MFMA_COUNTERS)} --kernel-trace`; per-launch medians (a launch issued as one dispatch "
           "per round of workgroups sums its dispatches' counters and durations). FLOP executed = "
           "`SQ_INSTS_VALU_MFMA_MOPS_*` x 512. Clock = `GRBM_GUI_ACTIVE` / 8 XCDs / kernel duration. "
           "MFMA busy = `SQ_VALU_MFMA_BUSY_CYCLES` / (cycles x 1024 SIMDs). Per-clock = FLOP / (cycles x 1024 "
           "SIMDs x dense FLOP per SIMD per clock: 1024 bf16, 2048 fp8), the fraction of the matrix cores' "
           "peak at the clock the chip ran. Peak fraction = FLOP / duration / (2.5 PFLOP/s bf16, 5.0 fp8), "
           "against the published 2.4 GHz figure.", "",
           "| kernel | dtype | launches | duration ms | TFLOP executed | clock GHz | MFMA busy | per-clock | "
           "of dense peak |", "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    machine = []
    for name in sorted(per):
        rows = per[name]
        med = {k: statistics.median(r[k] for r in rows) for k in ("flop", "ms", "clock_GHz", "mfma_busy",
                                                                 "per_clock", "peak_frac")}
        out.append(f"| `{name}` | {rows[0]['dtype']} | {len(rows)} | {med['ms']:.3f} | {med['flop'] / 1e12:.2f} | "
                   f"{med['clock_GHz']:.2f} | {med['mfma_busy']:.3f} | {med['per_clock']:.3f} | "
                   f"{med['peak_frac']:.3f} |")
        machine.append(f"mfma {name} dtype={rows[0]['dtype']} flop={med['flop']:.0f} clock_GHz={med['clock_GHz']:.3f} "
                       f"mfma_busy={med['mfma_busy']:.4f} per_clock={med['per_clock']:.4f}")
    out += ["", "Machine-readable (read by bench.py into `roofline`):", "", "```"] + machine + ["```", ""]
    return "\n".join(out)


def committed_mfma(config: str, kernel: str):
    """{mfma_busy, clock_GHz, mfma_per_clock, mfma_source} of `kernel` from the committed
    matrix-core summary, or None."""
    import re

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{PROFILE_PREFIX[config]}_mfma.md")
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(rf"^mfma {re.escape(kernel)} dtype=\w+ flop=\d+ clock_GHz=([\d.]+) mfma_busy=([\d.]+) "
                  rf"per_clock=([\d.]+)$", text, re.M)
    if not m:
        return None
    return {"clock_GHz": float(m.group(1)), "mfma_busy": float(m.group(2)), "mfma_per_clock": float(m.group(3)),
            "mfma_source": os.path.relpath(path, os.path.dirname(os.path.abspath(__file__)))}


# L1 -> L2 read pipeline counters, one --pmc pass each (with GRBM_GUI_ACTIVE and --kernel-trace)
MEMORY_PASSES = (("TCP_TCC_READ_REQ_sum", "TCP_TCC_READ_REQ_LATENCY_sum", "TCP_PENDING_STALL_CYCLES_sum",
                  "GRBM_GUI_ACTIVE"),
                 ("TCC_HIT_sum", "TCC_MISS_sum", "GRBM_GUI_ACTIVE"))
CUS = 256                           # MI355X compute units (one L1 each)


def memory_summary(directories, config: str, command: str) -> str:
    """Markdown: how each library GEMM kernel's loads move through the L1 (TCP) and the L2
    (TCC), from the MEMORY_PASSES runs (per-launch medians, each pass's values taken
    together):
    * L1 -> L2 read requests per launch, one per 128-byte line;
    * mean L2 read latency = TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ (cycles);
    * lines in flight per CU = TCP_TCC_READ_REQ_LATENCY / (cycles x 256 CUs): the average
      number of outstanding L1 misses per CU over the kernel (Little's law);
    * L1 pending-stall share = TCP_PENDING_STALL_CYCLES / (cycles x 256 CUs);
    * L2 hit rate = TCC_HIT / (TCC_HIT + TCC_MISS)."""
    import statistics

    per = {}
    for directory in directories:
        counters, durations = _per_dispatch(directory)
        for name, vals, ns, _ in _launches(counters, durations):
            if "GRBM_GUI_ACTIVE" not in vals or ns is None:
                continue
            cycles = vals["GRBM_GUI_ACTIVE"] / 8.0
            row = {}
            if "TCP_TCC_READ_REQ_sum" in vals and vals["TCP_TCC_READ_REQ_sum"] > 0:
                req, lat = vals["TCP_TCC_READ_REQ_sum"], vals["TCP_TCC_READ_REQ_LATENCY_sum"]
                row.update(req=req, latency=lat / req, inflight=lat / (cycles * CUS),
                           pending=vals["TCP_PENDING_STALL_CYCLES_sum"] / (cycles * CUS), cycles=cycles,
                           ms=ns / 1e6)
            if "TCC_HIT_sum" in vals and vals["TCC_HIT_sum"] + vals["TCC_MISS_sum"] > 0:
                row["hit"] = vals["TCC_HIT_sum"] / (vals["TCC_HIT_sum"] + vals["TCC_MISS_sum"])
            for k, v in row.items():
                per.setdefault(name, {}).setdefault(k, []).append(v)
    if not per:
        raise SystemExit(f"no library dispatches with memory counters in {directories}")
    passes = "; ".join(f"`--pmc {' '.join(p)} --kernel-trace`" for p in MEMORY_PASSES)
    out = [f"# L1 and L2 read pipeline per kernel: {config.upper()} (rocprofv3 TCP / TCC counters)", "",
           "Commands (from the repository root on the MI355X box):", "", "```", command.strip(), "```", "",
           f"One `bench.py --pmc-driver` pass per counter set ({passes}); per-launch medians (a launch issued as "
           "one dispatch per round of workgroups sums its dispatches). A request is one "
           "128-byte line from a CU's L1 (TCP) to the L2 (TCC). Latency = TCP_TCC_READ_REQ_LATENCY / "
           "TCP_TCC_READ_REQ, in cycles. Lines in flight per CU = TCP_TCC_READ_REQ_LATENCY / (cycles x 256 CUs), "
           "the mean number of outstanding L1 misses per CU (Little's law). Pending stall = "
           "TCP_PENDING_STALL_CYCLES / (cycles x 256 CUs). Cycles = GRBM_GUI_ACTIVE / 8 XCDs.", "",
           "| kernel | duration ms | L1->L2 requests (M) | GB at 128 B | mean L2 latency (cycles) | "
           "lines in flight per CU | L1 pending-stall share | L2 hit rate |",
           "|---|---:|---:|---:|---:|---:|---:|---:|"]
    machine = []

    def med(vals, k):
        return statistics.median(vals[k]) if k in vals else float("nan")

    for name in sorted(per):
        v = per[name]
        out.append(f"| `{name}` | {med(v, 'ms'):.3f} | {med(v, 'req') / 1e6:.1f} | {med(v, 'req') * 128 / 1e9:.2f} | "
                   f"{med(v, 'latency'):.0f} | {med(v, 'inflight'):.1f} | {med(v, 'pending'):.3f} | "
                   f"{med(v, 'hit'):.3f} |")
        machine.append(f"memory {name} requests={med(v, 'req'):.0f} latency={med(v, 'latency'):.1f} "
                       f"inflight={med(v, 'inflight'):.2f} hit={med(v, 'hit'):.4f}")
    out += ["", "Machine-readable:", "", "```"] + machine + ["```", ""]
    return "\n".join(out)


# --------------------------------------------------------------------------- CPU baseline


def cpu_threads() -> int:
    """Host threads of the CPU baseline: the job's CPU share (OMP_NUM_THREADS, 16 on the GPU
    box) when set, at most os.cpu_count()."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def time_cpu(run, reps: int = 3):
    """BASELINE's timing plan for the CPU leg: one untimed warmup, then `reps` timed
    repetitions; returns (median seconds, all timings)."""
    import statistics

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


# CPU-baseline sample rows for the secondary lines that carry one (whole blocks of 8)
SECONDARY_CPU_ROWS = {"c1": 512, "c4": 256}


def cpu_report(rows, n, med, times, threads, what, extra=""):
    """The cpu_baseline object: slots/s of a whole-block sample.  Every [N, V] operation is
    row-local and accept_len is block-local, so the sample's rate is the full batch's rate."""
    import torch

    return dict(value=rows / med, unit="slots/s", cores=threads, kind="port",
                sample=(f"numpy fp32 oracle (oracle/objective_ref.py), {what}, on {rows} of the {n} rows "
                        f"({rows // 8} whole blocks; every [N,V] op is row-local and accept_len block-local, so the "
                        f"sample's slots/s is the full batch's). 1 warmup + {len(times)} timed repetitions, median "
                        f"{med:.2f} s (all: {', '.join(f'{t:.2f}' for t in times)} s){extra}"),
                threads={"used": threads, "os_cpu_count": os.cpu_count(), "torch_get_num_threads": torch.get_num_threads(),
                         "cpu_model": cpu_model()})


def oracle_backward(ref, z, u, w, y, o, threads):
    """ce_kl_backward of the oracle over row chunks on `threads` host threads (row-local)."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor

    out = np.empty(z.shape, dtype=np.float32)

    def chunk(lo):
        hi = min(z.shape[0], lo + 16)
        out[lo:hi] = ref.ce_kl_backward(z[lo:hi], u[lo:hi], w[lo:hi], y[lo:hi], o.ce, o.kl, 1, dtype=np.float32)

    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(chunk, range(0, z.shape[0], 16)))
    return out


# --------------------------------------------------------------------------- C1


def workload_c1(device, args):
    import torch

    from nanospec_amd import objective, synthetic
    from nanospec_amd.config import Objective

    z, u, slots = synthetic.c1(device)
    n, v = z.shape
    o = Objective(block_size=8, gamma=4.0)

    def step():
        metrics, saved = objective.ce_kl_loss(z, u, slots, o)
        dl = objective.ce_kl_backward(saved)
        return metrics, dl

    # algorithmic bytes per slot: read z (bf16) + read u (bf16) + write dl (bf16)
    per_slot = 6 * v
    kernel_bytes = {
        "stream_stats": 4 * v * n,   # read z, u
        "stream_emit": 6 * v * n,    # read z, u, write dl
        # four workgroups per row, each keeping its quarter of z and u on chip: the whole
        # step's algorithmic bytes in one launch, each byte moved once
        "stream_group": 6 * v * n,
    }

    def cpu_baseline(rows):
        import numpy as np
        from threadpoolctl import threadpool_limits

        from oracle import objective_ref as ref

        rows = rows or 2048   # about 10-20 s of host work with warmup and 3 repetitions
        threads = cpu_threads()
        zs = z[:rows].float().cpu().numpy()
        us = u[:rows].float().cpu().numpy()
        w = slots.weights.reshape(-1)[:rows].cpu().numpy()
        y = slots.target_ids.reshape(-1)[:rows].cpu().numpy()
        vv = slots.valid.reshape(-1)[:rows].cpu().numpy()

        def run():
            ref.ce_kl_loss(zs, us, w.reshape(-1, 8), y.reshape(-1, 8), vv.reshape(-1, 8), o.ce, o.kl,
                           dtype=np.float32, chunk_rows=16, workers=threads)
            oracle_backward(ref, zs, us, w, y, o, threads)

        with threadpool_limits(limits=threads, user_api="blas"):
            med, times = time_cpu(run)
        return cpu_report(rows, n, med, times, threads,
                          f"ce_kl_loss + ce_kl_backward, row chunks on {threads} threads, V={v}")

    config = {"workload": "C1 logits-only: CE+KL+accept fwd + dlogits bwd over given bf16 [N,V] logits",
              "N": n, "V": v, "K": 8, "gamma": 4.0, "masked_rows": int((~slots.valid).sum()),
              "global_batch": n, "parallelism": "single GPU"}
    def ceilings():
        # library kernels with the same HBM access mix on the same tensors: two 2 GB
        # reads (stream_stats) and two reads plus one write (stream_emit)
        out = torch.empty_like(z)
        read2 = _time_ms(lambda: (torch.sum(z), torch.sum(u)))
        rw = _time_ms(lambda: torch.add(z, u, out=out))
        del out
        b = z.numel() * z.element_size()
        return {"method": "torch.sum(z), torch.sum(u) and torch.add(z, u, out=) on the C1 tensors",
                "read2_ms": read2, "read2_GBs": 2 * b / (read2 / 1e3) / 1e9,
                "read2_write1_ms": rw, "read2_write1_GBs": 3 * b / (rw / 1e3) / 1e9}

    return dict(step=step, n=n, per_slot_bytes=per_slot, per_slot_flops=None, kernel_bytes=kernel_bytes,
                kernel_flops={}, stream_kernels=("stream_stats", "stream_emit", "stream_group"), cpu_baseline=cpu_baseline,
                config=config, dtype="bf16", ceilings=ceilings,
                inputs={"draft_logits": z, "teacher_logits": u, "weights": slots.weights,
                        "target_ids": slots.target_ids, "valid": slots.valid})


# --------------------------------------------------------------------------- C2 / C3


def workload_head(device, args, which):
    import torch

    from nanospec_amd import head, synthetic
    from nanospec_amd.config import Objective

    gamma = 2.0 if which in ("c3", "c3s") else 4.0
    skip = which == "c3s"
    fp8 = None
    if which == "c4":
        from nanospec_amd import ops

        hidden, weight, markov, fp8, slots = synthetic.c4(device)
        teacher = None
    else:
        make = synthetic.c2 if which == "c2" else synthetic.c3
        hidden, weight, markov, teacher, slots = make(device)
    n, d = hidden.shape
    v = weight.shape[0]
    o = Objective(block_size=8, gamma=gamma)

    def step():
        u = teacher
        if fp8 is not None:
            # the fp8 head also forms each teacher row's log-sum-exp, so pass 1 reads no teacher
            xt, codes, scale = fp8
            u = ops.fp8_teacher_logits(xt, codes.view(torch.float8_e4m3fn), scale)
        metrics, saved = head.lm_head_ce_kl_loss(hidden, weight, u, slots, o, markov_logits=markov,
                                                 skip_masked_rows=skip)
        dh = head.lm_head_ce_kl_backward(saved)
        return metrics, dh

    gemm = 2.0 * n * v * d
    kernel_flops = {"head_stats": gemm, "head_emit": gemm, "dh_gemm": gemm}
    rows2 = n
    if skip:
        # pass 2 and the dh GEMM run on the rows whose dl is not all zero: here the supervised
        # ones (every row's statistics are finite); their executed work, not N's
        rows2 = int(((slots.valid.reshape(-1) != 0) | (slots.weights.reshape(-1) != 0)).sum())
        kernel_flops = {"head_stats": gemm, "head_emit": 2.0 * rows2 * v * d, "dh_gemm": 2.0 * rows2 * v * d}
    kernel_fp8_flops = {"fp8_head_gemm": gemm} if fp8 is not None else {}
    # byte streams of the epilogues (for the per-kernel GB/s report): pass 1 reads
    # Markov + teacher, pass 2 also writes dl; the dh GEMM reads dl
    kernel_bytes = {"head_stats": 4 * n * v, "head_emit": 6 * n * v, "dh_gemm": 2 * n * v}

    def cpu_baseline(rows):
        import numpy as np
        from threadpoolctl import threadpool_limits

        from oracle import objective_ref as ref

        rows = rows or (1024 if fp8 is not None else 1536)   # about 10-20 s with warmup and 3 repetitions
        threads = cpu_threads()
        w32 = weight.float().cpu().numpy()
        hs = hidden[:rows].float().cpu().numpy()
        ms = markov[:rows].float().cpu().numpy()
        wt = slots.weights.reshape(-1)[:rows].cpu().numpy()
        y = slots.target_ids.reshape(-1)[:rows].cpu().numpy()
        vv = slots.valid.reshape(-1)[:rows].cpu().numpy()
        fixed = None
        if fp8 is not None:
            xt, codes, scale = fp8
            xq = xt[:rows].float().cpu().numpy()
            wc = codes.cpu().numpy()
            sc = scale.cpu().numpy()
        else:
            us = teacher[:rows].float().cpu().numpy()

        def run():
            u = ref.fp8_linear(xq, wc, sc, dtype=np.float32) if fp8 is not None else us
            z = ref.lm_head_logits(hs, w32, ms, dtype=np.float32)
            ref.ce_kl_loss(z, u, wt.reshape(-1, 8), y.reshape(-1, 8), vv.reshape(-1, 8), o.ce, o.kl,
                           dtype=np.float32, chunk_rows=16, workers=threads)
            dl = oracle_backward(ref, z, u, wt, y, o, threads)
            ref.lm_head_backward(dl, w32, dtype=np.float32)

        with threadpool_limits(limits=threads, user_api="blas"):
            med, times = time_cpu(run)
            if fp8 is not None:
                # fp8_linear dequantises the whole weight on every call (ops.py:198-199), a cost per
                # batch, not per slot: time it alone and charge it once per N-row batch
                fixed, _ = time_cpu(lambda: ref.fp8_linear(xq[:8], wc, sc, dtype=np.float32), reps=1)
        extra = ""
        if fixed is not None:
            per_row = max(med - fixed, 1e-9) / rows
            med_full = fixed + per_row * n
            extra = (f"; the weight dequantisation ({fixed:.2f} s) is charged once per {n}-row batch: "
                     f"{med_full:.1f} s per batch")
            med = med_full * rows / n
        return cpu_report(rows, n, med, times, threads,
                          f"{'fp8_linear teacher head, ' if fp8 is not None else ''}LM-head GEMM (BLAS), "
                          f"ce_kl_loss, ce_kl_backward, dh GEMM; d={d}, V={v}; {threads} threads", extra)

    name = {"c2": "C2 full fused", "c3": "C3 long-batch", "c4": "C4 FP8 teacher head + full fused",
            "c3s": "C3 long-batch, pass 2 and dhidden on the rows with a nonzero dl only"}[which]
    config = {"workload": f"{name}: LM-head GEMM + Markov addend + CE+KL+accept fwd, dl + dhidden bwd",
              "N": n, "d": d, "V": v, "K": 8, "gamma": gamma, "global_batch": n, "seq_len": None,
              "parallelism": "single GPU"}
    if skip:
        config["skip_masked_rows"] = True
        config["pass2_rows"] = rows2
    def ceilings():
        # the vendor library's plain GEMM of the same shape (hipBLASLt through torch.mm):
        # the logits GEMM without any objective work, output written to HBM
        ht = hidden.t().contiguous()   # a contiguous right operand (no transposed view)
        mm = _time_ms(lambda: torch.mm(weight, ht))
        del ht
        out = {"method": "torch.mm(W_lm, hidden^T) (hipBLASLt), bf16, random operands", "gemm_ms": mm,
               "gemm_TFLOPs": gemm / (mm / 1e3) / 1e12}
        if fp8 is not None:
            out["fp8"] = fp8_ceilings(fp8)
        return out

    executed = gemm + 4.0 * rows2 * v * d if skip else None   # pass 1 on N rows, pass 2 and dh on rows2
    return dict(step=step, n=n, per_slot_bytes=None, per_slot_flops=4.0 * v * d, kernel_bytes=kernel_bytes,
                executed_flops_per_step=executed,
                kernel_flops=kernel_flops, kernel_fp8_flops=kernel_fp8_flops, cpu_baseline=cpu_baseline,
                config=config, dtype="bf16" if fp8 is None else "bf16+fp8", ceilings=ceilings,
                per_slot_fp8_flops=2.0 * v * d if fp8 is not None else None,
                inputs={"hidden": hidden, "lm_head_weight": weight, "markov_logits": markov,
                        "teacher_logits": teacher,
                        "teacher_hidden": fp8[0] if fp8 is not None else None,
                        "teacher_head_codes": fp8[1] if fp8 is not None else None,
                        "teacher_head_scales": fp8[2] if fp8 is not None else None,
                        "weights": slots.weights, "target_ids": slots.target_ids, "valid": slots.valid})


# --------------------------------------------------------------------------- C2X


def workload_c2x(device, args):
    """C2 with the path's neighbours included (train.py:271-310, 525-535; shard.py:
    318-330): final_norm (ops.rms_norm, weight ones as initialised, dspark.py:64-65) on a
    pre-norm N(0,1) input before the head and its backward fused after the dh GEMM; the
    Markov head in factored form at the reference rank (r = 256, config.py:26) instead of
    a dense [N, V] addend, with its backward (w2.grad copy, w1.grad index_add); the pooled
    tail and the gradient factor applied to the Markov and norm gradients."""
    import torch

    from nanospec_amd import head, ops, pooled, synthetic
    from nanospec_amd.config import Objective

    r = 256
    hidden, weight, markov, teacher, slots = synthetic.c2(device)
    del markov
    n, d = hidden.shape
    v = weight.shape[0]
    x = torch.randn((n, d), generator=torch.Generator(device=device).manual_seed(3002), device=device).bfloat16()
    norm_w = torch.ones(d, dtype=torch.bfloat16, device=device)
    norm_g = torch.zeros_like(norm_w)
    prev, w1, w2 = synthetic.markov_factors(n, v, r, 2002, device)
    if args.markov_skew > 0:
        # dropped anchor blocks give every slot the block's first id (dspark.py:120-127): a
        # fraction of the rows, spread over the batch, share one previous-token id
        hot = torch.randperm(n, generator=torch.Generator(device=device).manual_seed(4002), device=device)
        prev[hot[: int(args.markov_skew * n)]] = int(prev[0])
    mk = head.MarkovFactors(prev, w1, w2)
    w1_grad = torch.zeros_like(w1)
    w2_grad = torch.zeros_like(w2)
    o = Objective(block_size=8, gamma=4.0)
    del hidden

    def step():
        w1_grad.zero_()
        h, saved_norm = ops.rms_norm(x, norm_w, 1e-6)
        metrics, saved = head.lm_head_ce_kl_loss(h, weight, teacher, slots, o, markov=mk)
        dx = head.lm_head_ce_kl_backward(saved, markov_grads=(w1_grad, w2_grad),
                                         final_norm=(saved_norm, norm_w, norm_g))
        tail = pooled.pooled_tail(metrics)
        pooled.scale_gradients_((w1_grad, w2_grad, norm_g), tail.factor)
        return metrics, dx

    gemm_k = 2.0 * n * v * (d + r)
    kernel_flops = {"head_stats": gemm_k, "head_emit": gemm_k, "dh_gemm": gemm_k, "markov_dw2": 2.0 * n * v * r}
    kernel_bytes = {"head_stats": 2 * n * v, "head_emit": 4 * n * v, "dh_gemm": 2 * n * v,
                    "markov_dw2": 2 * n * v, "rms_norm_fwd": 6 * n * d}

    def cpu_baseline(rows):
        import numpy as np
        from threadpoolctl import threadpool_limits

        from oracle import objective_ref as ref

        rows = rows or 1024
        threads = cpu_threads()
        w32 = weight.float().cpu().numpy()
        w1n, w2n = w1.float().cpu().numpy(), w2.float().cpu().numpy()
        xs = x[:rows].float().cpu().numpy()
        wn = norm_w.float().cpu().numpy()
        pv = prev[:rows].cpu().numpy()
        us = teacher[:rows].float().cpu().numpy()
        wt = slots.weights.reshape(-1)[:rows].cpu().numpy()
        y = slots.target_ids.reshape(-1)[:rows].cpu().numpy()
        vv = slots.valid.reshape(-1)[:rows].cpu().numpy()

        def run():
            hs, inv, _ = ref.rms_norm(xs, wn, 1e-6)
            z = ref.lm_head_logits(hs, w32, dtype=np.float32) + ref.markov_logits(pv, w1n, w2n, dtype=np.float32)
            ref.ce_kl_loss(z, us, wt.reshape(-1, 8), y.reshape(-1, 8), vv.reshape(-1, 8), o.ce, o.kl,
                           dtype=np.float32, chunk_rows=16, workers=threads)
            dl = oracle_backward(ref, z, us, wt, y, o, threads)
            dh = ref.bf16_round(ref.lm_head_backward(dl, w32, dtype=np.float32))
            ref.rms_norm_backward(dh, xs, inv, wn)
            ref.markov_backward(dl, pv, w1n, w2n, dtype=np.float32)

        with threadpool_limits(limits=threads, user_api="blas"):
            med, times = time_cpu(run)
        return cpu_report(rows, n, med, times, threads,
                          f"rms_norm, LM-head + Markov GEMMs (BLAS), ce_kl_loss, ce_kl_backward, dh GEMM, rms_norm "
                          f"backward, Markov backward; d={d}, V={v}, r={r}; {threads} threads")

    config = {"workload": "C2X: C2 with final_norm around the head, the factored Markov head (r=256) fused "
                          "as a second K segment, and the pooled tail; fwd, dl + dx + final_norm / markov_w1 / "
                          "markov_w2 grads bwd, gradient factor applied",
              "N": n, "d": d, "V": v, "K": 8, "r": r, "gamma": 4.0, "markov_skew": args.markov_skew,
              "global_batch": n, "seq_len": None, "parallelism": "single GPU"}
    return dict(step=step, n=n, per_slot_bytes=None, per_slot_flops=4.0 * v * d + 6.0 * v * r,
                kernel_bytes=kernel_bytes, kernel_flops=kernel_flops, kernel_fp8_flops={},
                cpu_baseline=cpu_baseline, config=config, dtype="bf16", per_slot_fp8_flops=None,
                inputs={"pre_norm_hidden": x, "lm_head_weight": weight, "teacher_logits": teacher,
                        "previous": prev, "markov_w1": w1, "markov_w2": w2, "weights": slots.weights,
                        "target_ids": slots.target_ids, "valid": slots.valid})


WORKLOADS = {
    "c1": workload_c1,
    "c2x": workload_c2x,
    "c2": lambda dev, a: workload_head(dev, a, "c2"),
    "c3": lambda dev, a: workload_head(dev, a, "c3"),
    "c3s": lambda dev, a: workload_head(dev, a, "c3s"),
    "c4": lambda dev, a: workload_head(dev, a, "c4"),
}


def sample_sha256(t) -> str:
    """sha256 (first 16 hex digits) of about 64 Ki elements taken at a fixed stride from the
    flattened tensor: identifies the seeded inputs of a run without hashing gigabytes."""
    import hashlib

    import torch

    flat = t.reshape(-1)
    stride = max(1, flat.numel() // 65536)
    sample = flat[::stride].contiguous().cpu()
    if sample.dtype == torch.bool:
        sample = sample.to(torch.uint8)
    return hashlib.sha256(sample.view(torch.uint8).numpy().tobytes()).hexdigest()[:16]


def fp8_ceilings(fp8) -> dict:
    """The vendor library's fp8 GEMM of the teacher head's shape (torch._scaled_mm, hipBLASLt):
    x [N, d] e4m3 . W^T with W the same e4m3 codes [V, d], bf16 out.  Tensor-wise scales (a
    plain fp8 GEMM, no block scales), and the 1x128 / 128x128 block scales of ops.fp8_linear
    (ops.py:189-199) where the library takes them.  A form the library refuses is recorded
    with its error instead of a time."""
    import torch

    xt, codes, scale = fp8
    n, d = xt.shape
    v = codes.shape[0]
    flops = 2.0 * n * v * d
    a = xt.float().clamp(-448, 448).to(torch.float8_e4m3fn)
    b = codes.view(torch.float8_e4m3fn).t()          # [d, V], column-major as _scaled_mm wants
    one = torch.ones((), dtype=torch.float32, device=xt.device)
    forms = {
        "tensorwise": lambda: torch._scaled_mm(a, b, scale_a=one, scale_b=one, out_dtype=torch.bfloat16),
        "blockwise_1x128_128x128": lambda: torch._scaled_mm(
            a, b, scale_a=torch.ones((n, d // 128), dtype=torch.float32, device=xt.device),
            scale_b=scale.t(), out_dtype=torch.bfloat16),
    }
    out = {"method": "torch._scaled_mm(x_e4m3, W_e4m3^T) (hipBLASLt), bf16 out"}
    for name, fn in forms.items():
        try:
            ms = _time_ms(fn)
            out[name] = {"gemm_ms": ms, "gemm_TFLOPs": flops / (ms / 1e3) / 1e12,
                         "frac_fp8_peak": flops / (ms / 1e3) / 1e12 / FP8_PEAK_TFLOPS}
        except (RuntimeError, NotImplementedError, TypeError, ValueError) as e:
            out[name] = {"error": f"{type(e).__name__}: {str(e).splitlines()[0][:240]}"}
    del a
    return out


def _time_ms(fn, reps: int = 5) -> float:
    """Mean time of fn() on the current stream (one untimed call first)."""
    import torch

    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def pmc_driver(step, device):
    """One counter pass: one step, the calibration kernel (an elementwise fp32 negation
    that reads and writes CALIBRATION_BYTES), then two steps."""
    import torch

    step()
    torch.cuda.synchronize()
    src = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    print("pmc driver: done", flush=True)


def measure(wl, args, config_name):
    """Warmup, then exactly `args.steps` timed steps of workload `wl` between two device
    synchronisations; per-kernel means from the library's own HIP-event timer in the same
    window; the dominant kernel's roofline."""
    import torch

    from nanospec_amd import _lib

    step = wl["step"]
    # warmup: at least W steps and at least WARMUP_MIN_S of device time, so that the clocks
    # have left their idle state (C1, about 1 ms a step and arithmetic-bound, ran 1.156 ms a
    # kernel after 3 warmup steps and 1.063 ms after 300)
    warm = 0
    t_w = time.perf_counter()
    while warm < args.warmup or (time.perf_counter() - t_w < WARMUP_MIN_S and warm < WARMUP_MAX_STEPS):
        step()
        warm += 1
        if warm >= args.warmup:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    # timed window: exactly K steps between two device synchronisations.  The durations of
    # the kernels with a roofline (GEMMs, HBM streams) come from HIP events the library records
    # around each of their launches, on the stream the launch uses, inside this same window.
    # The short kernels between them run without events here: a pair of events costs a few
    # microseconds of the step (C1: 1.104 against 1.086 ms with every launch timed).
    fp8_flops = wl.get("kernel_fp8_flops", {})
    roofline_kernels = set(wl["kernel_flops"]) | set(wl["kernel_bytes"]) | set(fp8_flops)
    start_ev, stop_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with _lib.KernelTimer(only=roofline_kernels) as kt:
        start_ev.record()
        for _ in range(args.steps):
            step()
        stop_ev.record()
        torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start_ev.elapsed_time(stop_ev)
    ms_per_step = gpu_ms / args.steps
    n = wl["n"]
    value = n * args.steps / (gpu_ms / 1e3)
    kernels = {name: {"launches": c, "mean_ms": tot / max(c, 1), "window": "timed"}
               for name, (c, tot) in kt.times.items()}
    # the short kernels' means from a few more steps after the timed window, every launch timed
    detail_steps = max(3, args.steps // 4)
    with _lib.KernelTimer() as kd:
        for _ in range(detail_steps):
            step()
        torch.cuda.synchronize()
    for name, (c, tot) in kd.times.items():
        if name not in kernels:
            kernels[name] = {"launches": c, "mean_ms": tot / max(c, 1), "window": f"{detail_steps} steps after"}

    def roofline(kernel):
        k_ms = kernels[kernel]["mean_ms"]
        if kernel in wl["kernel_flops"] or kernel in fp8_flops:
            fp8 = kernel in fp8_flops
            peak = FP8_PEAK_TFLOPS if fp8 else BF16_PEAK_TFLOPS
            achieved = (fp8_flops if fp8 else wl["kernel_flops"])[kernel] / (k_ms / 1e3) / 1e12
            roof = {"bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
                    "frac": achieved / peak, "dtype": "fp8" if fp8 else "bf16"}
        else:
            achieved = wl["kernel_bytes"].get(kernel, 0) / (k_ms / 1e3) / 1e9
            roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": achieved / HBM_PEAK_GBS}
        roof["kernel"] = kernel
        roof["kernel_mean_ms"] = k_ms
        tr = committed_traffic(config_name, kernel)
        roof["traffic"] = tr[0] if tr else None
        if tr:
            roof["traffic_source"] = tr[1]
            # the bytes the kernel moves (counters), over this run's mean launch time: the
            # executed HBM rate beside the algorithmic one above
            roof["traffic_GBs"] = tr[0] / (k_ms / 1e3) / 1e9
            roof["traffic_frac_hbm"] = roof["traffic_GBs"] / HBM_PEAK_GBS
        mf = committed_mfma(config_name, kernel)
        if mf:
            roof.update(mf)
        return roof

    dominant = max(kt.times, key=lambda k: kt.times[k][1])
    roof = roofline(dominant)
    for name, info in kernels.items():
        if name in wl["kernel_bytes"]:
            info["algorithmic_GBs"] = wl["kernel_bytes"][name] / (info["mean_ms"] / 1e3) / 1e9
        if name in wl["kernel_flops"]:
            info["algorithmic_TFLOPs"] = wl["kernel_flops"][name] / (info["mean_ms"] / 1e3) / 1e12
            info["mfma_frac"] = info["algorithmic_TFLOPs"] / BF16_PEAK_TFLOPS
        if name in fp8_flops:
            info["algorithmic_TFLOPs"] = fp8_flops[name] / (info["mean_ms"] / 1e3) / 1e12
            info["mfma_frac_fp8"] = info["algorithmic_TFLOPs"] / FP8_PEAK_TFLOPS
    step_roof = {}
    if wl["per_slot_bytes"]:
        step_roof["algorithmic_GBs"] = wl["per_slot_bytes"] * n / (ms_per_step / 1e3) / 1e9
        step_roof["hbm_frac"] = step_roof["algorithmic_GBs"] / HBM_PEAK_GBS
    if wl["per_slot_flops"]:
        step_roof["algorithmic_TFLOPs"] = wl["per_slot_flops"] * n / (ms_per_step / 1e3) / 1e12
        # time the step would take at the dense peaks, over the measured step time
        ideal_s = wl["per_slot_flops"] * n / (BF16_PEAK_TFLOPS * 1e12)
        if wl.get("per_slot_fp8_flops"):
            ideal_s += wl["per_slot_fp8_flops"] * n / (FP8_PEAK_TFLOPS * 1e12)
        step_roof["mfma_frac"] = ideal_s / (ms_per_step / 1e3)
    if wl.get("executed_flops_per_step"):
        # the work the step runs when it skips rows (c3s): below N's algorithmic work
        step_roof["executed_TFLOPs"] = wl["executed_flops_per_step"] / (ms_per_step / 1e3) / 1e12
        step_roof["executed_mfma_frac"] = step_roof["executed_TFLOPs"] / BF16_PEAK_TFLOPS
    out = {"value": value, "unit": "slots/s", "steps": args.steps, "warmup": args.warmup, "warmup_steps_run": warm,
           "ms_per_step": ms_per_step, "dtype": wl["dtype"], "config": wl["config"], "roofline": roof,
           "step_roofline": step_roof, "kernels": kernels, "wall_s": wall}
    # every kernel the north star sets a target for: the HBM stream kernels and the GEMMs
    out["rooflines"] = {k: roofline(k) for k in kernels
                        if k in wl["kernel_flops"] or k in fp8_flops or k in wl.get("stream_kernels", ())}
    return out


def main():
    args = parse()
    if args.traffic_from:
        print(traffic_summary(args.traffic_from[0], args.traffic_from[1], args.config, args.command))
        return
    if args.stats_from:
        print(stats_summary(args.stats_from, args.config, args.command))
        return
    if args.mfma_from:
        print(mfma_summary(args.mfma_from, args.config, args.command))
        return
    if args.memory_from:
        print(memory_summary(args.memory_from, args.config, args.command))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}): the "
              "objective path is data-parallel over slots, so each GPU would run it on its own share of "
              "the anchor blocks and only the four pooled metric sums would be all-reduced; this library "
              "has no collectives.", file=sys.stderr)
        sys.exit(2)
    headline = args.config or "c2"
    if headline not in WORKLOADS:
        print(f"config {headline} is not available in this build", file=sys.stderr)
        sys.exit(2)

    import torch

    from nanospec_amd import _lib

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    _lib.load()
    wl = WORKLOADS[headline](device, args)
    if args.pmc_driver:
        pmc_driver(wl["step"], device)
        return

    res = measure(wl, args, headline)
    # practical ceilings measured with library kernels in this run (context for roofline)
    ceil = wl["ceilings"]() if "ceilings" in wl else None
    cpu = None
    if not args.no_cpu_baseline:
        cpu = wl["cpu_baseline"](args.cpu_rows)
    inputs_sha = {k: sample_sha256(t) for k, t in wl.get("inputs", {}).items() if t is not None}
    del wl
    torch.cuda.empty_cache()

    # the other configurations, in the same process, each with its own warmup and steps: C1
    # (the logit stream against HBM), C3 (the long batch), C4 (the fp8 teacher head) and C2X
    # (C2 with final_norm, the factored Markov head and the pooled tail)
    secondary = {}
    if args.config is None and not args.no_secondary:
        for name in ("c1", "c3", "c3s", "c4", "c2x"):
            wl2 = WORKLOADS[name](device, args)
            r2 = measure(wl2, args, name)
            if "ceilings" in wl2 and name != "c3s":   # c3s: the same shapes as c3
                r2["library_ceilings"] = wl2["ceilings"]()
            # the oracle on the host beside the logit stream and the fp8 teacher head too, on
            # smaller whole-block samples than the headline's (a few seconds each)
            if not args.no_cpu_baseline and name in SECONDARY_CPU_ROWS:
                r2["cpu_baseline"] = wl2["cpu_baseline"](SECONDARY_CPU_ROWS[name])
            r2["inputs_sha256"] = {k: sample_sha256(t) for k, t in wl2.get("inputs", {}).items() if t is not None}
            secondary[name] = r2
            del wl2
            torch.cuda.empty_cache()

    line = {
        "metric": METRIC,
        "value": res["value"],
        "unit": "slots/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": res["warmup_steps_run"],
        "warmup_min_s": WARMUP_MIN_S,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res["dtype"],
        "data": "synthetic (seeded; distributions of BASELINE.json configs)",
        "config": res["config"],
        "roofline": res["roofline"],
        "step_roofline": res["step_roofline"],
        "rooflines": res["rooflines"],
        "kernels": res["kernels"],
        "cpu_baseline": cpu,
        "library_ceilings": ceil,
        "wall_s": res["wall_s"],
        "inputs_sha256": inputs_sha,
        "secondary": secondary or None,
        "host": {"cpu_model": cpu_model(), "cpu_count": os.cpu_count()},
        "device": torch.cuda.get_device_name(device),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
