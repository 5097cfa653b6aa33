"""bench.py's roofline object on the CPU, for every kind of line it prints: the
HBM-bound decode sweeps, the MFMA-bound prefill sweeps (with the projections' operand
bytes) and the scaled-MFMA rate check (no operand bytes)."""

from __future__ import annotations

import bench


def test_roofline_hbm_line():
    r = {"value": 4000.0, "per_launch_bytes": 1e8, "per_launch_us": 25.0}
    roof = bench.roofline_of(r, False, "no such workload")
    assert roof["bound"] == "hbm" and roof["frac"] == 0.5 and roof["traffic"] is None
    assert roof["algorithmic_bytes_per_launch"] == 100000000 and roof["avg_launch_us"] == 25.0


def test_roofline_prefill_line_has_operand_bytes():
    r = {"tflops": 1250.0, "step_flops": 4e12, "launches": 4, "per_launch_bytes": 2e8, "per_launch_us": 800.0}
    roof = bench.roofline_of(r, True, "no such workload")
    assert roof["bound"] == "mfma" and roof["frac"] == 0.25
    assert roof["algorithmic_flops_per_launch"] == 10**12
    assert roof["algorithmic_operand_bytes_per_launch"] == 200000000


def test_roofline_mfma_rate_line():
    r = {"tflops": 4700.0, "step_flops": 4.3e13, "launches": 1, "per_launch_us": 9100.0}
    roof = bench.roofline_of(r, True, "mfma_scale_f32_16x16x128_f8f6f4")
    assert roof["frac"] == 0.94 and "algorithmic_operand_bytes_per_launch" not in roof
