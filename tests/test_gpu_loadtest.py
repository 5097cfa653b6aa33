"""The C++ manifest loader on the GPU: it binds mambo_quantize_mxfp8,
mambo_iq3s_prepare and mambo_iq3s_fp8_matmul through their runtime ABI manifests and
runs one projection on device 0 from the golden fixture (the reference test's M=9,
N=7, K=768 case, test_iq3_s_fp8.py:178-201): MXFP8 codes bit-exact, output within
rel-L2 1e-3 and the reference's elementwise rtol 5e-4 / atol 5e-3. The counterpart of
the reference's ABI-driven launch (tests/cpp/loadtest/loadtest.cpp:347-412)."""

from __future__ import annotations

import subprocess

import pytest

from conftest import GOLDEN
from test_abi_manifest import LOADTEST

pytestmark = pytest.mark.gpu


def test_loader_runs_a_projection_through_the_manifests(gpu, tmp_path):
    from mambo_amd import abi
    abi.write_manifests(tmp_path, library_path=str(abi.LIBRARY))
    assert LOADTEST.is_file(), f"{LOADTEST} is missing: run python -m mambo_amd.csrc.build"
    run = subprocess.run([str(LOADTEST), "--probe", str(GOLDEN / "matmul_small.npz"), "--abi-dir", str(tmp_path)],
                         capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    assert "ABI-driven projection passed for M=9 N=7 K=768" in run.stdout, run.stdout


def test_loader_probe_uses_the_in_tree_manifests(gpu):
    run = subprocess.run([str(LOADTEST), "--probe", str(GOLDEN / "matmul_small.npz"), "--abi-dir",
                          str(LOADTEST.parent / "abi")], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
