"""The reference's module paths and host-side behaviour, on the CPU (no launches).

Covers: the reference's import lines and `python -m mambo.utils.kernel_benchmark`
(test_iq3_s_fp8.py:15-21, kernel_benchmark.py:131-145), the E4M3 codebook against the
closed-form decoder (as test_iq3_s_fp8.py:71-81), the host GGUF reader behind
load_gguf_weight, the packed-weight cache's staleness rule, activation alignment copies,
and that a call the library rejects queues no work (split-K zero fill included)."""

from __future__ import annotations

import ctypes
import subprocess
import sys

import numpy as np
import pytest
import torch

from conftest import REPO, e4m3_values
from oracle import oracle
from test_tuning import write_gguf


def test_reference_import_lines_resolve_to_the_hip_path():
    # test_iq3_s_fp8.py:15-21, verbatim
    from mambo.kernels.iq3_s_fp8 import (  # noqa: F401
        iq3_s_fp8_table,
        iq3_s_table,
        launch_dequant_iq3_s,
        launch_iq3_s_fp8_matmul,
    )
    from mambo.kernels.quantize_fp8 import launch_quantize_fp8  # noqa: F401
    from mambo.utils.iq3_s_weight import prepare_iq3_s_fields  # noqa: F401
    from mambo.kernels.iq3_s_fp8 import BEST_CONFIGS, LARGE_TOKEN_THRESHOLD, make_benchmark_cases  # noqa: F401
    from mambo.kernels.iq3_s_fp8 import IQ3_S_BLOCK_BYTES, IQ3_S_BLOCK_VALUES, IQ3_S_SCALE_VALUES  # noqa: F401
    from mambo.utils.iq3_s_weight import IQ3SFields, _weight_dimensions, _weight_kernel_args  # noqa: F401
    from mambo.utils.iq3_s_weight import _large_weight_kernel_args  # noqa: F401
    from mambo.utils.kernel_benchmark import (  # noqa: F401
        BenchmarkCase, benchmark_main, load_gguf_weight, mini_benchmark, _BENCHMARKS)
    import mambo.kernels.iq3_s_fp8
    import mambo.kernels.quantize_fp8
    import mambo.utils.iq3_s_weight
    import mambo.utils.kernel_benchmark
    import mambo_amd.kernels.iq3_s_fp8
    import mambo_amd.kernels.quantize_fp8
    import mambo_amd.utils.iq3_s_weight
    import mambo_amd.utils.kernel_benchmark
    # one module object per path pair: state such as BEST_CONFIGS is shared
    assert mambo.kernels.iq3_s_fp8 is mambo_amd.kernels.iq3_s_fp8
    assert mambo.kernels.quantize_fp8 is mambo_amd.kernels.quantize_fp8
    assert mambo.utils.iq3_s_weight is mambo_amd.utils.iq3_s_weight
    assert mambo.utils.kernel_benchmark is mambo_amd.utils.kernel_benchmark
    assert LARGE_TOKEN_THRESHOLD == 32 and (IQ3_S_BLOCK_BYTES, IQ3_S_BLOCK_VALUES, IQ3_S_SCALE_VALUES) == (110, 256, 32)
    assert "iq3_s_fp8" in _BENCHMARKS


def test_kernel_benchmark_runs_as_a_module():
    run = subprocess.run([sys.executable, "-m", "mambo.utils.kernel_benchmark", "--help"], cwd=REPO,
                         capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    assert "iq3_s_fp8" in run.stdout and "--weight-name" in run.stdout and "--model" in run.stdout


def test_fp8_codebook_preserves_every_iq3_s_magnitude():
    """test_iq3_s_fp8.py:71-81 on the library's tables: each E4M3 byte of
    iq3_s_fp8_table decodes (closed-form OCP decoder) to the codebook magnitude, and
    with the sign bit set to its negation."""
    from mambo.kernels.iq3_s_fp8 import iq3_s_fp8_table, iq3_s_table
    raw, encoded = iq3_s_table(), iq3_s_fp8_table()
    assert raw.shape == encoded.shape == (512,) and raw.dtype == encoded.dtype == np.uint32
    magnitudes = raw.view(np.uint8).astype(np.float64)
    bits = encoded.view(np.uint8)
    dec = e4m3_values()
    np.testing.assert_array_equal(dec[bits], magnitudes)
    np.testing.assert_array_equal(dec[bits | 0x80], -magnitudes)


def test_read_block_matrix_and_its_errors(tmp_path):
    from mambo_amd.utils.gguf import read_block_matrix
    n, k = 5, 768
    raw = oracle.gen_iq3s(3, n, k // 256)
    path = tmp_path / "m.gguf"
    write_gguf(path, [("blk.0.attn_q.weight", [k, n], 21, raw.tobytes()),
                      ("blk.0.ffn_norm.weight", [16], 0, np.ones(16, np.float32).tobytes()),
                      ("bad.weight", [k, 2], 21, bytes(2 * 3 * 110))])
    got = read_block_matrix(path, "blk.0.attn_q.weight", "iq3_s")
    assert got.shape == (n, 3, 110) and got.dtype == np.uint8
    np.testing.assert_array_equal(got, raw)
    with pytest.raises(ValueError, match="no tensor named"):
        read_block_matrix(path, "blk.9.attn_q.weight", "iq3_s")
    with pytest.raises(ValueError, match="2D iq3_s"):
        read_block_matrix(path, "blk.0.ffn_norm.weight", "iq3_s")
    with pytest.raises(ValueError, match="2D q4_k"):
        read_block_matrix(path, "blk.0.attn_q.weight", "q4_k")


def test_packed_cache_follows_the_soa_fields():
    """The packed tile counts as current only for the field tensors it was built from,
    and only until one of them is written in place."""
    from dataclasses import replace

    from mambo_amd.utils.iq3_s_weight import PACKED_ONLY, IQ3SFields, fields_signature, packed_is_current
    blocks, n = 2, 16
    f = IQ3SFields(torch.zeros(blocks, n, dtype=torch.float16), torch.zeros(blocks, n, 16, dtype=torch.int32),
                   torch.zeros(blocks, n, 4, dtype=torch.int16), torch.zeros(blocks, n, 8, dtype=torch.int32),
                   torch.zeros(blocks, n, dtype=torch.int32))
    assert not packed_is_current(f)  # no tile yet
    g = replace(f, packed=torch.zeros(blocks * n * 110, dtype=torch.uint8))
    assert not packed_is_current(g)  # a tile of unknown origin is rebuilt
    object.__setattr__(g, "packed_from", fields_signature(g))
    assert packed_is_current(g)
    g.d[0, 3] = 1.0  # write through the field
    assert not packed_is_current(g)
    object.__setattr__(g, "packed_from", fields_signature(g))
    g.qs.view(torch.uint8)[1, 2, 3] = 7  # write through a view of a field
    assert not packed_is_current(g)
    object.__setattr__(g, "packed_from", fields_signature(g))
    h = replace(g, scales=g.scales.clone())  # a field replaced, the stale tile carried over
    assert not packed_is_current(h)
    assert packed_is_current(replace(g, packed=g.packed.clone()))  # same fields, another tile
    p = replace(f, packed=torch.zeros(8, dtype=torch.uint8), packed_from=PACKED_ONLY)
    p.d[0, 0] = 2.0  # placeholder fields of a packed-only weight do not matter
    assert packed_is_current(p)



def test_release_soa_fields_keeps_only_the_tile():
    """release_soa_fields: with a current packed tile, the five SoA fields become
    zero-stride placeholders of the same shapes and dtypes (their tensors are freed once
    nothing else holds them), the tile is kept and stays current, and the standalone
    decoder, which reads the fields, refuses the weight."""
    import gc
    import weakref

    from mambo_amd.kernels.iq3_s_fp8 import launch_dequant_iq3_s
    from mambo_amd.utils.iq3_s_weight import (IQ3SFields, fields_signature, has_soa_fields, packed_is_current,
                                              release_soa_fields)
    blocks, n = 3, 32
    f = IQ3SFields(torch.ones(blocks, n, dtype=torch.float16), torch.ones(blocks, n, 16, dtype=torch.uint32),
                   torch.ones(blocks, n, 4, dtype=torch.uint16), torch.ones(blocks, n, 8, dtype=torch.int32),
                   torch.ones(blocks, n, dtype=torch.uint32), torch.zeros(blocks * n * 110, dtype=torch.uint8))
    object.__setattr__(f, "packed_from", fields_signature(f))
    shapes = [(t.shape, t.dtype) for t in (f.d, f.qs, f.qh, f.signs, f.scales)]
    refs = [weakref.ref(t) for t in (f.d, f.qs, f.qh, f.signs, f.scales)]
    tile = f.packed
    assert has_soa_fields(f) and packed_is_current(f)
    assert release_soa_fields(f) is f
    gc.collect()
    assert all(r() is None for r in refs)  # the SoA tensors are gone
    assert f.packed is tile and packed_is_current(f) and not has_soa_fields(f)
    for t, (shape, dtype) in zip((f.d, f.qs, f.qh, f.signs, f.scales), shapes):
        assert t.shape == shape and t.dtype == dtype and all(st == 0 for st in t.stride())
    assert release_soa_fields(f) is f and f.packed is tile  # a second release changes nothing
    with pytest.raises(ValueError, match="SoA fields"):
        launch_dequant_iq3_s(f)

def test_activation_rows_are_copied_only_when_misaligned():
    from mambo_amd.kernels.iq3_s_fp8 import _aligned_rows
    base = torch.arange(4 * 96, dtype=torch.uint8).reshape(4, 96)
    ok = base[:, :64]  # row stride 96: 16- and 8-byte aligned
    assert _aligned_rows(ok, 16) is ok
    odd = torch.arange(4 * 68, dtype=torch.uint8).reshape(4, 68)[:, :64]  # row stride 68
    assert _aligned_rows(odd, 4) is odd
    for align in (8, 16):
        c = _aligned_rows(odd, align)
        assert c is not odd and c.is_contiguous() and torch.equal(c, odd)
    shifted = torch.arange(4 * 96 + 1, dtype=torch.uint8)[1:].reshape(4, 96)  # base address + 1
    c = _aligned_rows(shifted, 8)
    assert c.data_ptr() % 8 == 0 and torch.equal(c, shifted)
    strided = base[:, ::2]  # column stride 2
    c = _aligned_rows(strided, 16)
    assert c.stride() == (48, 1) and torch.equal(c, strided)


def test_rejected_projection_queues_no_zero_fill():
    """A K-split call that a later check rejects (tiled kernel: scale rows must be 8-byte
    aligned) returns that check's ValueError; the zero fill of the output, which would
    run first, is never queued (on this GPU-less host a queued kernel would fail with
    a runtime error instead)."""
    from mambo_amd import _native
    lib = _native.lib()
    cfg = _native.GemmConfig.from_dict({"kernel": _native.GEMM_TILED, "waves": 4, "split_k": 2, "tile_m": 64,
                                        "tile_n": 64})
    m, n, blocks = 64, 64, 4
    assert lib.mambo_gemm_check_config(m, n, blocks, ctypes.byref(cfg)) == 0
    # dummy device addresses: nothing is dereferenced before the checks reject the call
    xv, xs, packed, out = 0x10000, 0x20004, 0x30000, 0x40000
    rc = lib.mambo_iq3s_fp8_matmul(xv, blocks * 256, xs, blocks * 8, m, packed, n, blocks, out, n,
                                   ctypes.byref(cfg), None)
    assert rc == _native.MAMBO_ERR_VALUE, lib.mambo_last_error()
    assert b"8-byte aligned" in lib.mambo_last_error()
    # a configuration with no build (stream kernel, 3 waves) under a K split: rejected
    # before the zero fill as well
    bad = _native.GemmConfig.from_dict({"kernel": _native.GEMM_STREAM, "waves": 3, "split_k": 2})
    rc = lib.mambo_iq3s_fp8_matmul(xv, blocks * 256, 0x20000, blocks * 8, 1, packed, n, blocks, out, n,
                                   ctypes.byref(bad), None)
    assert rc == _native.MAMBO_ERR_VALUE and b"waves" in lib.mambo_last_error()
