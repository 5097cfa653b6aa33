"""The autotuner end to end on the GPU (kernel_benchmark.py:27-141 semantics): every
candidate of the search space runs, the winner's output matches the oracle, the tuned
table is written and then used by launch_iq3_s_fp8_matmul; and a weight read from a GGUF
file goes through the same path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_l2
from oracle import oracle
from test_tuning import write_gguf

pytestmark = pytest.mark.gpu


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def test_autotune_search_winner_and_table(gpu, tmp_path, monkeypatch):
    from mambo_amd.kernels import iq3_s_fp8
    from mambo_amd.utils.kernel_benchmark import mini_benchmark, synthetic_weight, write_tuned_table
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    n, k = 256, 2048
    step(f"synthetic weight {n}x{k}, tune M=4 and M=64")
    raw = synthetic_weight(n, k, seed=11)
    cases = iq3_s_fp8.make_benchmark_cases(raw, tokens=(4, 64), rotate_bytes=4 << 20)
    assert all(c.rotation == -(-(4 << 20) // (n * k // 256 * 110)) for c in cases)
    results = mini_benchmark(cases, quiet=True)
    assert [r.key for r in results] == [iq3_s_fp8.tuned_key(n, k, 4), iq3_s_fp8.tuned_key(n, k, 64)]
    for case, r in zip(cases, results):
        assert r.best in list(case.search_space)
        assert not r.failures, r.failures[:3]
        assert len(r.successes) == len(case.search_space)
        assert r.event_us > 0 and r.mean_us > 0 and r.batched_us > 0
        # the library default is timed, and only a 3% faster candidate replaces it
        assert r.default_us is not None and r.default_of == case.default
        assert r.is_default or r.tuner_us <= 0.97 * r.default_us
    # the winners reproduce the oracle
    fields = prepare_iq3_s_fields(raw)
    raw_np = raw.cpu().numpy()
    for m, r in zip((4, 64), results):
        x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
        xv, xs = oracle.quantize_mxfp8(x)
        step(f"winner M={m}: {r.best}")
        out = iq3_s_fp8.launch_iq3_s_fp8_matmul(torch.from_numpy(xv).to(gpu), torch.from_numpy(xs).to(gpu), fields,
                                                config=r.best)
        torch.cuda.synchronize()
        assert rel_l2(out.cpu().numpy(), oracle.iq3s_fp8_matmul(xv, xs, raw_np)) <= 1e-3
    # the table is written and then consulted by the launcher's config selection
    path = tmp_path / "tuned.json"
    write_tuned_table(results, path, "gfx950")
    monkeypatch.setattr(iq3_s_fp8, "TUNED_PATH", path)
    iq3_s_fp8._tuned_table.cache_clear()
    try:
        assert iq3_s_fp8.select_config(4, n, k, arch="gfx950") == results[0].best
        assert iq3_s_fp8.select_config(64, n, k, arch="gfx950") == results[1].best
    finally:
        iq3_s_fp8._tuned_table.cache_clear()


def test_gguf_weight_through_the_projection(gpu, tmp_path):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    from mambo_amd.utils.kernel_benchmark import load_gguf_weight
    n, k = 40, 1024
    raw = oracle.gen_iq3s(21, n, k // 256)
    path = tmp_path / "m.gguf"
    write_gguf(path, [("output_norm.weight", [16], 0, np.ones(16, np.float32).tobytes()),
                      ("blk.0.attn_q.weight", [k, n], 21, raw.tobytes())])
    step("load GGUF tensor, prepare, quantize, matmul")
    w = load_gguf_weight(path, "blk.0.attn_q.weight", "iq3_s")
    assert tuple(w.shape) == (n, k // 256, 110) and w.is_cuda
    np.testing.assert_array_equal(w.cpu().numpy(), raw)
    x = np.random.default_rng(5).standard_normal((3, k)).astype(np.float32)
    xq, xs = launch_quantize_fp8(torch.from_numpy(x).to(gpu))
    out = launch_iq3_s_fp8_matmul(xq, xs, prepare_iq3_s_fields(w))
    torch.cuda.synchronize()
    expected = oracle.iq3s_fp8_matmul(xq.cpu().numpy(), xs.cpu().numpy(), raw)
    assert rel_l2(out.cpu().numpy(), expected) <= 1e-3
    with pytest.raises(ValueError, match="no tensor named"):
        load_gguf_weight(path, "missing", "iq3_s")
    with pytest.raises(ValueError, match="2D iq3_s"):
        load_gguf_weight(path, "output_norm.weight", "iq3_s")


@pytest.mark.timeout(480)
def test_benchmark_command_on_a_gguf_file(gpu, tmp_path, capsys):
    """The reference's command line, verbatim (kernel_benchmark.py:131-141:
    `iq3_s_fp8 --model M --weight-name NAME`), through the reference's module path, on a
    GGUF file written here; then `python -m mambo.utils.kernel_benchmark ... --write-table`
    in a process of its own, whose table holds a valid entry for each tuned shape."""
    import ctypes
    import json
    import subprocess
    import sys

    from conftest import REPO
    from mambo.kernels import iq3_s_fp8
    from mambo_amd import _native
    from mambo.utils.kernel_benchmark import benchmark_main
    n, k = 96, 2048
    path = tmp_path / "model.gguf"
    write_gguf(path, [("blk.3.ffn_down.weight", [k, n], 21, oracle.gen_iq3s(33, n, k // 256).tobytes())])
    step("benchmark_main iq3_s_fp8 --model ... --weight-name blk.3.ffn_down.weight")
    results = benchmark_main(["iq3_s_fp8", "--model", str(path), "--weight-name", "blk.3.ffn_down.weight"])
    text = capsys.readouterr().out
    assert [r.case for r in results] == [f"M=4 N={n} K={k}", f"M=128 N={n} K={k}"]
    for r in results:
        assert f"{r.case}: best_config=" in text
        assert r.mean_us > 0 and r.batched_us > 0 and r.event_us > 0 and not r.failures
    assert "(warmup=5, iterations=20), candidates=" in text
    table = tmp_path / "tuned.json"
    step("python -m mambo.utils.kernel_benchmark ... --write-table")
    run = subprocess.run([sys.executable, "-m", "mambo.utils.kernel_benchmark", "iq3_s_fp8", "--model", str(path),
                          "--weight-name", "blk.3.ffn_down.weight", "--tokens", "4", "32",
                          "--write-table", "--table", str(table)],
                         cwd=REPO, capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stderr[-2000:]
    assert f"M=4 N={n} K={k}: best_config=" in run.stdout
    written = json.loads(table.read_text())
    assert set(written) == {"gfx950"}
    for key, cfg in written["gfx950"].items():  # shapes whose default won have no entry
        assert key in (iq3_s_fp8.tuned_key(n, k, 4), iq3_s_fp8.tuned_key(n, k, 32)), key
        c = _native.GemmConfig.from_dict(cfg)
        assert _native.lib().mambo_gemm_check_config(int(key.split("@")[1]), n, k // 256, ctypes.byref(c)) == 0


@pytest.mark.timeout(300)
def test_sweep_tuner_on_one_layer(gpu, tmp_path, capsys):
    """`--sweep llama8b --layers 1`: every candidate of each of the layer's four launch
    shapes runs inside the replayed layer and matches the library default's outputs (a
    mismatch would be a failure), and the table gets an entry exactly for the shapes whose
    winner beat the default."""
    import ctypes
    import json

    from mambo_amd import _native
    from mambo_amd.kernels import iq3_s_fp8
    from mambo_amd.utils.kernel_benchmark import benchmark_main
    shapes = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]  # q/k/v, o, gate/up, down
    table = tmp_path / "tuned.json"
    step("benchmark_main iq3_s_fp8 --sweep llama8b --layers 1 --tokens 1 16 --steps 3 --write-table")
    results = benchmark_main(["iq3_s_fp8", "--sweep", "llama8b", "--layers", "1", "--tokens", "1", "16",
                              "--steps", "3", "--write-table", "--table", str(table)])
    text = capsys.readouterr().out
    assert [r.key for r in results] == [iq3_s_fp8.tuned_key(n, k, m) for m in (1, 16) for n, k in shapes]
    written = json.loads(table.read_text())["gfx950"]
    for r, (m, (n, k)) in zip(results, [(m, s) for m in (1, 16) for s in shapes]):
        assert f"{r.case}: best_config=" in text
        # progress while searching: a line every 10 candidates and one after the last
        total = len(iq3_s_fp8.gemm_search_space(m, n, k))
        assert f"[tune] M={m} N={n} K={k}: candidate {total}/{total}, 0 failed, best so far" in text
        if total >= 10:
            assert f"[tune] M={m} N={n} K={k}: candidate 10/{total}," in text
        assert not r.failures, r.failures[:3]
        assert len(r.successes) == len(iq3_s_fp8.gemm_search_space(m, n, k))
        assert r.best in iq3_s_fp8.gemm_search_space(m, n, k)
        assert r.default_of == iq3_s_fp8.default_config(m) and r.default_us is not None
        assert r.mean_us > 0 and r.batched_us > 0 and r.event_us > 0 and r.tuner_us > 0
        assert r.is_default or r.tuner_us <= 0.99 * r.default_us
        if r.is_default:
            assert r.key not in written
        else:
            assert written[r.key] == r.best
            c = _native.GemmConfig.from_dict(r.best)
            assert _native.lib().mambo_gemm_check_config(m, n, k // 256, ctypes.byref(c)) == 0
