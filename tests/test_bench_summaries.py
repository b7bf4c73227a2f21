"""Host logic of bench.py's profile summaries: the matrix-core and L1/L2 read-pipeline figures
computed from rocprofv3 CSV files, checked on small hand-made files with known answers."""

import csv
import os

import pytest

import bench

HEAD = "void ns::(anonymous namespace)::head_kernel<0, unsigned short, 0>(ns::(anonymous namespace)::HeadParams)"
OTHER = "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda>(int)"


def _write_pass(directory, dispatches):
    """dispatches: [(dispatch id, kernel name, duration ns, {counter: value})]"""
    os.makedirs(directory, exist_ok=True)
    with open(os.path.join(directory, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for d, name, _, counters in dispatches:
            for c, v in counters.items():
                w.writerow([d, name, c, v])
    with open(os.path.join(directory, "run_kernel_trace.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        for d, name, ns, _ in dispatches:
            w.writerow([d, name, 1000, 1000 + ns])


def _machine(text, prefix, kernel):
    for line in text.splitlines():
        if line.startswith(f"{prefix} {kernel} "):
            return dict(kv.split("=") for kv in line.split()[2:])
    raise AssertionError(f"no {prefix} line for {kernel}")


def test_memory_summary_little_law(tmp_path):
    # 2 ms at 8 XCDs x 1.5e6 cycles: 1.5e6 cycles.  256 CUs x 64 lines in flight x 1.5e6 cycles
    # of latency summed, over 1e8 requests: mean latency 245.76 cycles, 64 lines per CU.
    cycles = 1.5e6
    req, lat = 1.0e8, 64 * 256 * cycles
    p1 = [(5, HEAD, 2_000_000, {"TCP_TCC_READ_REQ_sum": req, "TCP_TCC_READ_REQ_LATENCY_sum": lat,
                                "TCP_PENDING_STALL_CYCLES_sum": 0.25 * 256 * cycles, "GRBM_GUI_ACTIVE": 8 * cycles}),
          (6, OTHER, 1000, {"TCP_TCC_READ_REQ_sum": 7.0, "TCP_TCC_READ_REQ_LATENCY_sum": 7.0,
                            "TCP_PENDING_STALL_CYCLES_sum": 0.0, "GRBM_GUI_ACTIVE": 8.0})]
    p2 = [(5, HEAD, 2_000_000, {"TCC_HIT_sum": 3.0e8, "TCC_MISS_sum": 1.0e8, "GRBM_GUI_ACTIVE": 8 * cycles})]
    _write_pass(tmp_path / "a", p1)
    _write_pass(tmp_path / "b", p2)
    text = bench.memory_summary([str(tmp_path / "a"), str(tmp_path / "b")], "c2", "cmd")
    m = _machine(text, "memory", "head_stats")
    assert float(m["requests"]) == req
    assert float(m["latency"]) == pytest.approx(lat / req, abs=0.05)
    assert float(m["inflight"]) == pytest.approx(64.0, abs=0.005)
    assert float(m["hit"]) == pytest.approx(0.75, abs=1e-4)
    assert "| `head_stats` | 2.000 | 100.0 | 12.80 |" in text   # duration, M requests, GB at 128 B
    assert "0.250" in text                                    # pending-stall share
    assert "neg" not in text                                  # torch kernels are not summarised


def test_mfma_summary_clock_and_busy(tmp_path):
    # 10 ms at 1.5 GHz: 1.5e7 cycles per XCD.  MFMA busy on half of 1024 SIMDs' cycles; the
    # executed FLOP at 0.4 of the per-clock bf16 peak.
    cycles = 1.5e7
    flop = 0.4 * cycles * 1024 * 1024
    d = [(3, HEAD, 10_000_000, {"SQ_INSTS_VALU_MFMA_MOPS_BF16": flop / 512, "SQ_INSTS_VALU_MFMA_MOPS_F8": 0.0,
                                "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * cycles * 1024, "GRBM_GUI_ACTIVE": 8 * cycles})]
    _write_pass(tmp_path / "m", d)
    text = bench.mfma_summary(str(tmp_path / "m"), "c2", "cmd")
    m = _machine(text, "mfma", "head_stats")
    assert m["dtype"] == "bf16"
    assert float(m["clock_GHz"]) == pytest.approx(1.5, abs=1e-3)
    assert float(m["mfma_busy"]) == pytest.approx(0.5, abs=1e-4)
    assert float(m["per_clock"]) == pytest.approx(0.4, abs=1e-4)


DH = "void ns::(anonymous namespace)::dh_kernel(ns::(anonymous namespace)::BwdParams)"


def test_launch_split_into_rounds_counts_once(tmp_path):
    # two steps; each issues the dh GEMM as three dispatches (one per round) between other kernels:
    # the traffic and matrix-core figures are per launch (sums over the three), not per dispatch
    cycles = 1.0e6
    def dh(d, k):
        return (d, DH, 1_000_000, {"SQ_INSTS_VALU_MFMA_MOPS_BF16": 1.0e6 * k, "SQ_INSTS_VALU_MFMA_MOPS_F8": 0.0,
                                   "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * cycles * 1024, "GRBM_GUI_ACTIVE": 8 * cycles})
    step1 = [(1, HEAD, 2_000_000, {"SQ_INSTS_VALU_MFMA_MOPS_BF16": 5.0e6, "SQ_INSTS_VALU_MFMA_MOPS_F8": 0.0,
                                   "SQ_VALU_MFMA_BUSY_CYCLES": 0.0, "GRBM_GUI_ACTIVE": 16 * cycles}),
             dh(2, 1), dh(3, 2), dh(4, 3)]
    step2 = [(5, OTHER, 1000, {"SQ_INSTS_VALU_MFMA_MOPS_BF16": 0.0, "SQ_INSTS_VALU_MFMA_MOPS_F8": 0.0,
                               "SQ_VALU_MFMA_BUSY_CYCLES": 0.0, "GRBM_GUI_ACTIVE": 8.0}),
             dh(6, 1), dh(7, 2), dh(8, 3)]
    _write_pass(tmp_path / "m", step1 + step2)
    text = bench.mfma_summary(str(tmp_path / "m"), "c3", "cmd")
    m = _machine(text, "mfma", "dh_gemm")
    assert float(m["flop"]) == pytest.approx(512 * 6.0e6)          # 1 + 2 + 3 million MOPS per launch
    assert float(m["clock_GHz"]) == pytest.approx(1.0, abs=1e-3)   # 3e6 cycles over 3 ms
    assert float(m["mfma_busy"]) == pytest.approx(0.5, abs=1e-4)
    assert "| `dh_gemm` | bf16 | 2 | 3.000 |" in text                # two launches of 3 ms

    # traffic: FETCH_SIZE per launch is the sum of its dispatches (KiB; calibration 1 GiB)
    for sub, counter in (("f", "FETCH_SIZE"), ("w", "WRITE_SIZE")):
        rows = [(1, HEAD, 10, {counter: 100.0}), (2, DH, 10, {counter: 10.0}), (3, DH, 10, {counter: 20.0}),
                (4, OTHER, 10, {counter: 1024.0 * 1024.0}), (5, DH, 10, {counter: 30.0}),
                (6, DH, 10, {counter: 30.0}), (7, HEAD, 10, {counter: 100.0})]
        _write_pass(tmp_path / sub, rows)
    text = bench.traffic_summary(str(tmp_path / "f"), str(tmp_path / "w"), "c3", "cmd")
    t = _machine(text, "traffic", "dh_gemm")
    # launches of 30 and 60 KiB: median 45 KiB
    assert float(t["fetch_bytes"]) == pytest.approx(45 * 1024)
    assert float(t["write_bytes"]) == pytest.approx(45 * 1024)
    assert float(_machine(text, "traffic", "head_stats")["fetch_bytes"]) == pytest.approx(100 * 1024)


def test_stats_summary_launch_column(tmp_path):
    d = tmp_path / "s"
    os.makedirs(d)
    with open(d / "run_kernel_stats.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        w.writerow([DH, 6, 60_000_000, 10_000_000, 60.0])
        w.writerow([HEAD, 2, 40_000_000, 20_000_000, 40.0])
    _write_pass(d, [(1, HEAD, 1, {}), (2, DH, 1, {}), (3, DH, 1, {}), (4, DH, 1, {}),
                    (5, HEAD, 1, {}), (6, DH, 1, {}), (7, DH, 1, {}), (8, DH, 1, {})])
    text = bench.stats_summary(str(d), "c3", "cmd")
    assert "| dh_gemm | 6 | 2 | 60.000 | 10.0000 | 30.0000 | 60.0 |" in text
    assert "| head_stats | 2 | 2 | 40.000 | 20.0000 | 20.0000 | 40.0 |" in text
    # one dispatch per launch everywhere: the plain table
    os.remove(d / "run_kernel_trace.csv")
    _write_pass(d, [(1, HEAD, 1, {}), (2, DH, 1, {}), (3, OTHER, 1, {}), (4, HEAD, 1, {}), (5, DH, 1, {})])
    with open(d / "run_kernel_stats.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"])
        w.writerow([DH, 2, 20_000_000, 10_000_000, 50.0])
    text = bench.stats_summary(str(d), "c2", "cmd")
    assert "| dh_gemm | 2 | 20.000 | 10.0000 | 50.0 |" in text
