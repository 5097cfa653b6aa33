"""The per-point profile summary (mambo_amd/utils/rocprof_summary.py points) end to end on
the CPU, over synthetic rocprofv3 CSVs of a two-point bench run: the trace cut into each
point's timed replays, traffic per launch from FETCH_SIZE / WRITE_SIZE scaled by the copy
calibration, MFMA busy of the MFMA-bound point, and the traffic records bench.py reads."""

from __future__ import annotations

import csv
import json

from mambo_amd.utils import rocprof_summary

STEPS, WARMUP = 2, 1
# (workload, m, launches per step, dispatches per step: launches plus fills)
POINTS = [("decode sweep, M=1", 1, 3, 3), ("llama3-8b prefill sweep, M=2048", 2048, 2, 2)]


def bench_line() -> dict:
    def roof(m, launches):
        if m >= 128:
            return {"bound": "mfma", "frac": 0.2, "unit": "TFLOP/s", "avg_launch_us": 10.0,
                    "algorithmic_flops_per_launch": 10**9, "algorithmic_operand_bytes_per_launch": 1000}
        return {"bound": "hbm", "frac": 0.5, "unit": "GB/s", "avg_launch_us": 1.0,
                "algorithmic_bytes_per_launch": 4000}
    (w0, m0, l0, _), (w1, m1, l1, _) = POINTS
    return {"steps": STEPS, "warmup": WARMUP, "ms_per_step": 0.004,
            "config": {"workload": w0, "m": m0, "launches_per_step": l0}, "roofline": roof(m0, l0),
            "value": 1.0, "unit": "GB/s",
            "points": [{"workload": w1, "m": m1, "launches_per_step": l1, "ms_per_step": 0.03,
                        "roofline": roof(m1, l1), "value": 1.0, "unit": "TFLOP/s"}]}


def write_trace(path):
    """Per point: input set-up, the eager step, a check copy, the check replay, a compare,
    then W + K replays; each GEMM dispatch lasts 1 us (decode) or 10 us (prefill)."""
    rows, t = [], 0
    def add(name, dur_ns):
        nonlocal t
        rows.append((name, t, t + dur_ns))
        t += dur_ns + 100
    for _, m, _, d in POINTS:
        dur = 10000 if m >= 128 else 1000
        add("randn", 500)
        for _ in range(d):
            add("void gemm_stream_kernel<1>", dur)
        add("copy", 500)
        for _ in range(d):
            add("void gemm_stream_kernel<1>", dur)
        add("allclose", 500)
        for _ in range((WARMUP + STEPS) * d):
            add("void gemm_stream_kernel<1>", dur)
    with open(path / "t_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writerows(rows)


def write_counters(path, counter_values: dict):
    """One eager step and one timed step per point (bench.py --no-graph --steps 1
    --warmup 0), every dispatch with the given counter values, set-up kernels between."""
    rows, did = [], 0
    def add(name, values):
        nonlocal did
        for counter, value in values.items():
            rows.append((did, name, counter, value))
        did += 1
    for _, _, _, d in POINTS:
        add("randn", {c: 1.0 for c in counter_values})
        for _ in range(2 * d):
            add("void gemm_stream_kernel<1>", counter_values)
    path.mkdir()
    with open(path / "c_counter_collection.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writerows(rows)


def test_points_report_end_to_end(tmp_path):
    (tmp_path / "line.json").write_text(json.dumps(bench_line()) + "\n")
    write_trace(tmp_path)
    write_counters(tmp_path / "fetch", {"FETCH_SIZE": 3.0})
    write_counters(tmp_path / "write", {"WRITE_SIZE": 1.0})
    # copy calibration: 2048 bytes per FETCH_SIZE unit, 1024 per WRITE_SIZE unit
    for name, counter, value in (("cf", "FETCH_SIZE", 512.0), ("cw", "WRITE_SIZE", 1024.0)):
        (tmp_path / name).mkdir()
        with open(tmp_path / name / "c_counter_collection.csv", "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
            w.writerow([0, "copy_bytes_kernel", counter, value])
    write_counters(tmp_path / "mfma", {"SQ_VALU_MFMA_BUSY_CYCLES": 4096.0, "SQ_INSTS_VALU_MFMA_MOPS_F8": 2 * 10**9 / 512,
                                      "GRBM_GUI_ACTIVE": 64.0})
    out = tmp_path / "summary.md"
    rocprof_summary.main(["points", "--bench-json", str(tmp_path / "line.json"), "--bench-command", "b",
                          "--plain-json", str(tmp_path / "line.json"), "--trace", str(tmp_path),
                          "--fetch", str(tmp_path / "fetch"), "--write", str(tmp_path / "write"),
                          "--calib-fetch", str(tmp_path / "cf"), "--calib-write", str(tmp_path / "cw"),
                          "--copy-bytes", str(1 << 20), "--mfma", str(tmp_path / "mfma"), "--out", str(out),
                          "--out-dir", str(tmp_path)])
    text = out.read_text()
    # decode point: 3 dispatches of 1 us per step -> 0.003 ms, 3 x 4000 bytes / 3 us = 4 GB/s
    assert "| 8B M=1 | 3 | 1.000 |" in text or "| 70B M=1 | 3 | 1.000 |" in text
    rec = json.loads(out.with_suffix(".json").read_text())
    assert abs(rec[0]["kernel_ms_per_step"] - 0.003) < 1e-12 and abs(rec[1]["gemm_us_per_launch"] - 10.0) < 1e-9
    assert abs(rec[0]["frac_kernel"] - 4000 * 3 / 3e-6 / 1e9 / 8000) < 1e-12
    # traffic: per dispatch 3 x 2048 + 1 x 1024 bytes, 3 dispatches over 3 launches
    t0 = json.loads((tmp_path / "traffic_llama8b_m1.json").read_text())
    assert t0["workload"] == POINTS[0][0] and t0["traffic_bytes_per_launch"] == 3 * 2048 + 1024
    assert t0["traffic_over_algorithmic"] == (3 * 2048 + 1024) / 4000
    # MFMA busy: 4096 / (64 / 8 XCDs x 1024 SIMDs) = 50%; executed F8 flops 2 x per dispatch
    assert "| 8B M=2048 | 50.0% | 2.000 |" in text
