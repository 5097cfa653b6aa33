"""The oracle's command-line tool against the protocol of the reference's oracle
executable (tests/cpp/reference/ggml_reference.cpp:192-268,317-343) and the reference's
contract tests for it (test_reference_fixture.py:24-66): the NPY-over-stdout packet
and its metadata, the CPU arrays against the oracle library and numpy, timing on
stderr only with --benchmark, and the rejected inputs (truncated or trailing stdin,
NaN, unknown tensor or type, malformed arguments)."""

from __future__ import annotations

import subprocess

import numpy as np
import pytest

from conftest import make_synthetic_iq3_s
from oracle import oracle
from test_tuning import write_gguf

WEIGHT = "blk.1.attn_qkv.weight"


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    oracle.build()
    path = tmp_path_factory.mktemp("cli") / "model.gguf"
    raw = make_synthetic_iq3_s(24, 768, seed=0x3F8)
    write_gguf(path, [("token_embd.weight", [16], 0, np.ones(16, np.float32).tobytes()),
                      (WEIGHT, [768, 24], 21, raw.tobytes())])
    return path, raw


def run_cli(args, stdin: bytes):
    return subprocess.run([str(oracle.CLI_PATH), *args], input=stdin, capture_output=True, check=False, timeout=120)


@pytest.mark.parametrize("m", [1, 8])
def test_matmul_packet_and_arrays(model, m):
    path, raw = model
    x = np.random.Generator(np.random.PCG64(20261013)).standard_normal((m, 768), dtype=np.float32)
    arrays, header = oracle.cli_matmul(path, WEIGHT, x)
    assert header["tensor_name"] == WEIGHT and header["ggml_type"] == "iq3_s" and header["backend"] == "cpu"
    assert header["shape_ggml_ne_order"] == [768, 24] and header["row_bytes"] == 3 * 110
    assert header["tensor_bytes"] == 24 * 3 * 110
    blob = path.read_bytes()
    off = header["data_offset_absolute"]
    np.testing.assert_array_equal(np.frombuffer(blob, np.uint8, 24 * 330, off).reshape(24, 3, 110), raw)
    w = oracle.dequant_iq3s(raw)
    np.testing.assert_array_equal(arrays["dequant_rows"], w[:4])
    # the reference harness's bound for this array (compute_reference_gguf.py:242)
    np.testing.assert_allclose(arrays["ggml_dequant_f64"], (x.astype(np.float64) @ w.astype(np.float64).T)
                               .astype(np.float32), rtol=1e-6, atol=2e-5)
    xv, xs = oracle.quantize_mxfp8(x)
    np.testing.assert_allclose(arrays["mxfp8_f64"], oracle.iq3s_fp8_matmul(xv, xs, raw), rtol=1e-6, atol=2e-5)


def test_benchmark_reports_timing_only_on_stderr(model):
    path, _ = model
    x = np.ones((1, 768), dtype=np.float32)
    run = run_cli(["--op", "matmul", "--model", str(path), "--weight", WEIGHT, "--m", "1", "--benchmark",
                   "--benchmark-iters", "2"], x.tobytes())
    assert run.returncode == 0, run.stderr.decode(errors="replace")
    assert not run.stdout
    assert b"benchmark backend=cpu op=matmul" in run.stderr
    assert b"iterations=2 mean_us=" in run.stderr
    assert b" batched_us=" in run.stderr and b" event_us=" in run.stderr


def test_rejects_truncated_and_trailing_stdin(model):
    path, _ = model
    args = ["--op", "matmul", "--model", str(path), "--weight", WEIGHT, "--m", "1"]
    for stdin in (b"\0", np.ones(769, np.float32).tobytes()):
        run = run_cli(args, stdin)
        assert run.returncode != 0
        assert b"input size mismatch" in run.stderr
        assert not run.stdout
    bad = np.ones((1, 768), np.float32)
    bad[0, 7] = np.nan
    run = run_cli(args, bad.tobytes())
    assert run.returncode != 0 and b"NaN or infinity" in run.stderr and not run.stdout


@pytest.mark.parametrize("args,message", [
    (["--op", "matmul", "--weight", WEIGHT, "--m", "1"], b"missing required argument"),
    (["--op", "conv", "--model", "{model}", "--weight", WEIGHT, "--m", "1"], b"unsupported op"),
    (["--op", "matmul", "--model", "{model}", "--weight", "missing", "--m", "1"], b"tensor not found"),
    (["--op", "matmul", "--model", "{model}", "--weight", "token_embd.weight", "--m", "1"],
     b"unsupported ggml tensor type"),
    (["--op", "matmul", "--model", "{model}", "--weight", WEIGHT, "--m", "0"], b"M must be a positive integer"),
    (["--op", "matmul", "--model", "{model}", "--weight", WEIGHT, "--m", "1", "--m", "2"], b"more than once"),
    (["--op", "matmul", "--model", "{model}", "--weight", WEIGHT, "--m", "1", "--benchmark-iters", "3"],
     b"requires --benchmark"),
    (["--op", "matmul", "--model", "{model}", "--weight", WEIGHT, "--m", "1", "--dequant-rows", "25"],
     b"cannot exceed"),
    (["--op", "matmul", "--model", "{model}", "--weight", WEIGHT, "--m", "1", "--fast"], b"unknown argument"),
])
def test_rejects_bad_invocations(model, args, message):
    path, _ = model
    run = run_cli([a.replace("{model}", str(path)) for a in args], np.ones(768, np.float32).tobytes())
    assert run.returncode == 1 and message in run.stderr, run.stderr
    assert run.stderr.startswith(b"mambo_oracle_cli: ") and not run.stdout


def test_help_and_not_a_gguf(tmp_path):
    oracle.build()
    run = run_cli(["--help"], b"")
    assert run.returncode == 0 and b"--op matmul --model PATH" in run.stderr and not run.stdout
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + bytes(60))
    run = run_cli(["--op", "matmul", "--model", str(bad), "--weight", WEIGHT, "--m", "1"], b"")
    assert run.returncode == 1 and b"not a GGUF file" in run.stderr
