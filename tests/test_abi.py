"""The C ABI library (no GPU): it loads, exports every entry point include/mambo_hip.h
declares, and rejects bad arguments with the documented status codes before touching
the device; the Python layer maps them to the reference's exception types."""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from conftest import REPO

HEADER = REPO / "include" / "mambo_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mambo_\w+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    from mambo_amd import _native
    lib = _native.lib()
    names = declared_symbols()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), f"{name} declared in mambo_hip.h but not exported"
    assert set(names) == set(_native.SIGNATURES), "ctypes declarations must match the header"
    assert lib.mambo_abi_version() == 100
    assert lib.mambo_build_arch() == b"gfx950"


def test_status_codes_and_last_error():
    from mambo_amd import _native
    lib = _native.lib()
    # K not divisible by 32 -> MAMBO_ERR_VALUE before any device work
    rc = lib.mambo_quantize_mxfp8(None, 1, 4, 100, 100, None, 100, None, 4, None)
    assert rc == _native.MAMBO_ERR_VALUE
    assert b"K divisible by 32" in lib.mambo_last_error()
    rc = lib.mambo_quantize_mxfp8(None, 7, 4, 64, 64, None, 64, None, 2, None)
    assert rc == _native.MAMBO_ERR_VALUE and b"dtype" in lib.mambo_last_error()
    with pytest.raises(ValueError, match="dtype"):
        _native.check(rc)
    rc = lib.mambo_iq3s_prepare(None, 4, 1, 110, 110, 1, None, None, None, None, None, None, None)
    assert rc == _native.MAMBO_ERR_VALUE
    # the quantize + matmul entry point validates dtype and pointers before device work
    rc = lib.mambo_iq3s_matmul_quantize_grouped(None, 7, 256, 1, None, 1, 1, None, None, 256, None, 8, None)
    assert rc == _native.MAMBO_ERR_VALUE and b"dtype" in lib.mambo_last_error()
    rc = lib.mambo_iq3s_matmul_quantize_grouped(None, _native.DTYPE_BF16, 256, 1, None, 1, 1, None, None, 256, None,
                                                8, None)
    assert rc == _native.MAMBO_ERR_VALUE and b"null" in lib.mambo_last_error()
    assert lib.mambo_iq3s_packed_bytes(0, 3) == 0
    assert lib.mambo_iq3s_packed_bytes(17, 3) == 2 * 3 * 1760
    assert lib.mambo_iq3s_packed_bytes(4096, 16) == 4096 * 16 * 110  # byte-preserving


def test_gemm_config_defaults_and_validation():
    from mambo_amd import _native
    lib = _native.lib()
    cfg = _native.GemmConfig()
    assert lib.mambo_gemm_default_config(1, 4096, 16, ctypes.byref(cfg)) == 0
    assert cfg.kernel == _native.GEMM_STREAM and cfg.waves in (1, 2, 4, 6, 8, 12, 16) and 1 <= cfg.split_k <= 16
    # 8 waves with at least 4 blocks each (or small grids), 4 for large grids of short K,
    # 16 for tiny grids, K split only below 512 waves; runs of round(tiles / 512) tiles
    # per workgroup (tile_n = 16 rows per tile)
    for n, blocks, waves, split, tile_n in (
            (28672, 32, 8, 1, 64), (8192, 32, 8, 1, 16), (8192, 112, 8, 1, 16), (10240, 32, 8, 1, 16),
            (57344, 32, 8, 1, 112), (28672, 16, 4, 1, 64), (4096, 16, 8, 1, 16), (1024, 32, 16, 1, 16),
            (1024, 16, 8, 1, 16), (64, 64, 16, 2, 16), (14336, 16, 8, 1, 32)):
        big = _native.GemmConfig()
        assert lib.mambo_gemm_default_config(1, n, blocks, ctypes.byref(big)) == 0
        assert (big.waves, big.split_k, big.tile_n) == (waves, split, tile_n), (n, blocks, big.as_dict())
    for tile_n, rc in ((0, 0), (48, 0), (16 * 4096, 0), (24, _native.MAMBO_ERR_VALUE), (-16, _native.MAMBO_ERR_VALUE)):
        c = _native.GemmConfig.from_dict({"kernel": _native.GEMM_STREAM, "waves": 4, "split_k": 1, "tile_n": tile_n})
        assert lib.mambo_gemm_check_config(1, 64, 4, ctypes.byref(c)) == rc, tile_n
    bad = _native.GemmConfig.from_dict({"kernel": _native.GEMM_STREAM, "waves": 5, "split_k": 1})
    assert lib.mambo_gemm_check_config(1, 64, 4, ctypes.byref(bad)) == _native.MAMBO_ERR_VALUE
    bad = _native.GemmConfig.from_dict({"kernel": _native.GEMM_STREAM, "waves": 4, "split_k": 9})
    assert lib.mambo_gemm_check_config(1, 64, 4, ctypes.byref(bad)) == _native.MAMBO_ERR_VALUE
    ok = _native.GemmConfig.from_dict({"kernel": _native.GEMM_STREAM, "waves": 8, "split_k": 4})
    assert lib.mambo_gemm_check_config(1, 64, 4, ctypes.byref(ok)) == 0
    ok = _native.GemmConfig.from_dict({"kernel": _native.GEMM_DENSE, "waves": 8, "split_k": 4})
    assert lib.mambo_gemm_check_config(1, 64, 4, ctypes.byref(ok)) == 0
    bad = _native.GemmConfig.from_dict({"kernel": _native.GEMM_TILED, "waves": 8, "split_k": 1})
    assert lib.mambo_gemm_check_config(1, 64, 4, ctypes.byref(bad)) == _native.MAMBO_ERR_VALUE
    ok = _native.GemmConfig.from_dict({"kernel": _native.GEMM_TILED, "waves": 4, "split_k": 1, "tile_m": 128,
                                       "tile_n": 128})
    assert lib.mambo_gemm_check_config(256, 64, 4, ctypes.byref(ok)) == 0
    for bad_fields in ({"tile_m": 96}, {"waves": 2, "tile_n": 32}, {"tile_n": 96}, {"split_k": 5},
                       {"waves": 16, "tile_n": 256}):
        bad = _native.GemmConfig.from_dict({"kernel": _native.GEMM_TILED, "waves": 4, "split_k": 1, "tile_m": 128,
                                            "tile_n": 128, **bad_fields})
        assert lib.mambo_gemm_check_config(256, 64, 4, ctypes.byref(bad)) == _native.MAMBO_ERR_VALUE, bad_fields
    split = _native.GemmConfig.from_dict({"kernel": _native.GEMM_TILED, "waves": 4, "split_k": 4, "tile_m": 128,
                                          "tile_n": 128})
    assert lib.mambo_gemm_check_config(256, 64, 4, ctypes.byref(split)) == 0
    # 256 tokens: built for 8 or 16 waves of 16 weight rows only; 16 waves only there
    for fields, rc in (({"waves": 8, "tile_n": 128}, 0), ({"waves": 16, "tile_n": 256}, 0),
                       ({"waves": 4, "tile_n": 64}, _native.MAMBO_ERR_VALUE),
                       ({"waves": 8, "tile_n": 256}, _native.MAMBO_ERR_VALUE),
                       ({"waves": 16, "tile_n": 512}, _native.MAMBO_ERR_VALUE)):
        c = _native.GemmConfig.from_dict({"kernel": _native.GEMM_TILED, "split_k": 1, "tile_m": 256, **fields})
        assert lib.mambo_gemm_check_config(2048, 4096, 16, ctypes.byref(c)) == rc, fields
    # dense default: 32 tokens per workgroup above 16 tokens; tiles per workgroup by grid size
    for m, n, tile_m, tile_n in ((16, 8192, 16, 32), (16, 57344, 16, 64), (48, 57344, 32, 64), (32, 1024, 32, 16)):
        c = _native.GemmConfig()
        assert lib.mambo_gemm_default_config(m, n, 32, ctypes.byref(c)) == 0
        assert (c.kernel, c.tile_m, c.tile_n, c.waves) == (_native.GEMM_DENSE, tile_m, tile_n, 4), (m, n, c.as_dict())
    # 17-32 tokens: 32-token tiles of 4 x 16 weight rows, K split toward ~512 workgroups
    # (at most 4 splits of at least 8 blocks) unless the grid stays under half the CUs
    for m, n, blocks, split in ((32, 57344, 32, 1), (32, 8192, 32, 4), (32, 10240, 32, 4), (24, 8192, 32, 4),
                                (17, 28672, 16, 2), (32, 8192, 112, 4), (32, 4096, 16, 2)):
        c = _native.GemmConfig()
        assert lib.mambo_gemm_default_config(m, n, blocks, ctypes.byref(c)) == 0
        assert (c.kernel, c.tile_m, c.tile_n, c.waves, c.split_k) == (_native.GEMM_TILED, 32, 64, 4, split), \
            (m, n, blocks, c.as_dict())
        assert lib.mambo_gemm_check_config(m, n, blocks, ctypes.byref(c)) == 0
    for fields, rc in (({"tile_m": 32, "waves": 4}, 0), ({"tile_m": 32, "waves": 16}, _native.MAMBO_ERR_VALUE),
                       ({"tile_m": 48, "waves": 4}, _native.MAMBO_ERR_VALUE)):
        c = _native.GemmConfig.from_dict({"kernel": _native.GEMM_DENSE, "split_k": 1, **fields})
        assert lib.mambo_gemm_check_config(32, 4096, 16, ctypes.byref(c)) == rc, fields
    # prefill default: 256 x 256 x 16 waves when every round of its grid (one workgroup
    # per CU) fills at least 7/8 of the CUs (and the tokens are padded by at most 1/8 more
    # than with 128-token tiles), else 256 x 128 x 8 under the same rule, else
    # 128 x 128 x 8 when that gives every CU a workgroup (padding at most 1/8 over 64-token
    # tiles), else 64 x 128 x 8; 256 x 128 x 8 also where both 256-token grids fill their
    # rounds and its rounds are at least 8% fuller; on long K (>= 48 blocks) 256 x 128 x 8
    # with a K split that fills one round when there is one (at least 16 blocks per
    # split), else the 128-token tile with K split until the grid covers the chip twice
    for m, n, blocks, tile, split in ((2048, 4096, 32, (256, 128, 8), 1), (2048, 4096, 16, (256, 128, 8), 1),
                                      (2048, 4096, 56, (256, 128, 8), 1), (8192, 4096, 16, (256, 256, 16), 1),
                                      (8192, 14336, 32, (256, 256, 16), 1),
                                      (512, 8192, 32, (128, 128, 8), 1), (512, 57344, 32, (256, 256, 16), 1),
                                      (512, 28672, 16, (256, 256, 16), 1), (2048, 6144, 16, (128, 128, 8), 1),
                                      (2048, 10240, 32, (128, 128, 8), 1), (8192, 10240, 32, (256, 256, 16), 1),
                                      (256, 8192, 32, (64, 128, 8), 1), (64, 57344, 32, (64, 128, 8), 1),
                                      (128, 57344, 32, (128, 128, 8), 1), (384, 57344, 32, (128, 128, 8), 1),
                                      (192, 57344, 32, (64, 128, 8), 1), (256, 8192, 112, (256, 128, 8), 4),
                                      (512, 8192, 112, (256, 128, 8), 2), (2048, 8192, 112, (256, 256, 16), 1),
                                      (512, 4096, 56, (128, 128, 8), 3), (768, 4096, 56, (128, 128, 8), 3),
                                      (1024, 4096, 56, (256, 128, 8), 2), (768, 8192, 112, (128, 128, 8), 2),
                                      (2048, 28672, 16, (256, 128, 8), 1), (1536, 28672, 16, (256, 256, 16), 1),
                                      (1024, 57344, 32, (256, 128, 8), 1), (128, 8192, 112, (128, 128, 8), 7)):
        c = _native.GemmConfig()
        assert lib.mambo_gemm_default_config(m, n, blocks, ctypes.byref(c)) == 0
        assert (c.kernel, c.tile_m, c.tile_n, c.waves, c.split_k) == (_native.GEMM_TILED, *tile, split), \
            (m, n, blocks, c.as_dict())
        assert lib.mambo_gemm_check_config(m, n, blocks, ctypes.byref(c)) == 0
    # moderate M on a long K: the tiled default splits K to fill the chip
    c = _native.GemmConfig()
    assert lib.mambo_gemm_default_config(64, 8192, 112, ctypes.byref(c)) == 0
    assert c.kernel == _native.GEMM_TILED and c.split_k > 1, c.as_dict()
    # block-diagonal activations up to M=4, dense up to 63, tiled from 64 - except for
    # few weight rows below 256 tokens, where the tiled grid stays small
    for m, n, kernel in ((1, 8192, _native.GEMM_STREAM), (4, 8192, _native.GEMM_STREAM),
                         (5, 8192, _native.GEMM_DENSE), (16, 8192, _native.GEMM_DENSE),
                         (63, 8192, _native.GEMM_DENSE), (64, 8192, _native.GEMM_TILED),
                         (2048, 8192, _native.GEMM_TILED), (128, 1024, _native.GEMM_DENSE),
                         (256, 1024, _native.GEMM_TILED)):
        c = _native.GemmConfig()
        assert lib.mambo_gemm_default_config(m, n, 32, ctypes.byref(c)) == 0
        assert c.kernel == kernel, (m, n, c.as_dict())
        assert lib.mambo_gemm_check_config(m, n, 32, ctypes.byref(c)) == 0


def test_codebook_exports_match_python_tables():
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import iq3_s_fp8_table, iq3_s_table
    out = np.zeros(512, dtype=np.uint32)
    assert _native.lib().mambo_iq3s_fp8_grid(out.ctypes.data) == 0
    np.testing.assert_array_equal(out, iq3_s_fp8_table())
    assert _native.lib().mambo_iq3s_grid(out.ctypes.data) == 0
    np.testing.assert_array_equal(out, iq3_s_table())


def test_python_api_validation_without_gpu():
    import torch
    from mambo_amd.kernels.iq3_s_fp8 import (launch_dequant_iq3_s, launch_iq3_s_fp8_matmul,
                                             launch_iq3_s_fp8_matmul_grouped, m_bucket, select_config)
    from mambo_amd.utils.iq3_s_weight import IQ3SFields
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    with pytest.raises(ValueError):
        launch_quantize_fp8(torch.zeros(4, 33))
    with pytest.raises(ValueError):
        launch_quantize_fp8(torch.zeros(4, 32, dtype=torch.float16))
    with pytest.raises(ValueError):
        launch_quantize_fp8(torch.zeros(4, 64))  # not on a GPU
    with pytest.raises(ValueError):
        prepare_iq3_s_fields(torch.zeros(4, 2, 109, dtype=torch.uint8))
    with pytest.raises(ValueError):
        prepare_iq3_s_fields(torch.zeros(0, 2, 110, dtype=torch.uint8))
    with pytest.raises(TypeError):
        launch_iq3_s_fp8_matmul(torch.zeros(1, 256, dtype=torch.uint8), torch.zeros(1, 8, dtype=torch.uint8),
                                "not prepared")
    with pytest.raises(TypeError):
        launch_dequant_iq3_s(object())

    def fields(n, blocks):  # field shapes only; validation runs before any launch
        return IQ3SFields(torch.zeros(blocks, n, dtype=torch.float16), torch.zeros(blocks, n, 16, dtype=torch.int32),
                          torch.zeros(blocks, n, 4, dtype=torch.int16), torch.zeros(blocks, n, 8, dtype=torch.int32),
                          torch.zeros(blocks, n, dtype=torch.int32))
    xv, xs = torch.zeros(1, 512, dtype=torch.uint8), torch.zeros(1, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match="share K"):
        launch_iq3_s_fp8_matmul_grouped(xv, xs, [fields(16, 2), fields(16, 1)])
    with pytest.raises(ValueError, match="between 1 and 4"):
        launch_iq3_s_fp8_matmul_grouped(xv, xs, [fields(16, 2)] * 5)
    with pytest.raises(ValueError, match="between 1 and 4"):
        launch_iq3_s_fp8_matmul_grouped(xv, xs, [])
    with pytest.raises(TypeError):
        launch_iq3_s_fp8_matmul_grouped(xv, xs, [fields(16, 2), "not prepared"])
    with pytest.raises(ValueError, match="x_scales"):
        launch_iq3_s_fp8_matmul_grouped(xv, xs[:, :8], [fields(16, 2)])
    with pytest.raises(RuntimeError, match="no tuned config"):
        select_config(4, 4096, 4096, arch="gfx942")
    assert select_config(4, 4096, 4096, arch="gfx950")["kernel"] == 0  # the library picks the family
    assert [m_bucket(m) for m in (1, 2, 3, 4, 5, 16, 17, 2048)] == [1, 2, 4, 4, 8, 16, 32, 2048]


def test_split_table_is_exact():
    """(1+2s)(2l+1) = 2*E4M3(hi) + 2*E4M3(lo) for every scale nibble and grid level, hi is
    the product rounded to 4 significant bits with ties to even, |lo| <= 16."""
    from fractions import Fraction
    from mambo_amd import _native
    from oracle import oracle
    table = np.zeros(64, dtype=np.uint32)
    assert _native.lib().mambo_iq3s_split_table(table.ctypes.data) == 0
    dec = oracle.e4m3_decode_all()  # float value of every E4M3 byte

    def rne4(p):  # nearest value with 4 significant bits, ties to the even one
        step = 1 << max(0, p.bit_length() - 4)
        lo, hi = p // step * step, (p // step + 1) * step
        if p - lo != hi - p:
            return lo if p - lo < hi - p else hi
        return lo if (lo // step) % 2 == 0 else hi

    for s in range(16):
        for lvl in range(8):
            w = lvl >> 2
            hb = int(table[4 * s + w] >> (8 * (lvl & 3))) & 0xFF
            lb = int(table[4 * s + 2 + w] >> (8 * (lvl & 3))) & 0xFF
            p = (1 + 2 * s) * (2 * lvl + 1)
            hi, lo = Fraction(float(dec[hb])) * 2, Fraction(float(dec[lb])) * 2
            assert hb < 0x80 and hi == rne4(p), (s, lvl, hb, hi)
            assert hi + lo == p and abs(lo) <= 16, (s, lvl, hi, lo)


def test_chain_validation_without_gpu():
    """mambo_iq3s_fp8_matmul_chain rejects bad arguments before touching the device."""
    from mambo_amd import _native
    lib = _native.lib()
    sync = (ctypes.c_uint32 * _native.CHAIN_SYNC_WORDS)()
    one = (_native.ChainLaunch * 1)()
    one[0].x, one[0].x_dtype, one[0].count, one[0].ldx = 16, _native.DTYPE_MXFP8, 1, 256
    one[0].xs, one[0].ldxs, one[0].blocks = 16, 8, 1
    one[0].proj[0] = _native.Projection(16, 16, 16, 16)
    sp = ctypes.addressof(sync)
    cases = [
        (lambda: lib.mambo_iq3s_fp8_matmul_chain(1, one, 0, None, sp, None), "count must be in"),
        (lambda: lib.mambo_iq3s_fp8_matmul_chain(5, one, 1, None, sp, None), "1..4 tokens"),
        (lambda: lib.mambo_iq3s_fp8_matmul_chain(1, one, 1, None, None, None), "null pointer"),
    ]
    for call, text in cases:
        assert call() == _native.MAMBO_ERR_VALUE
        assert text in lib.mambo_last_error().decode()
    for field, value, text in (("x_dtype", 7, "x_dtype"), ("ldx", 100, "row stride"), ("blocks", 0, "K blocks"),
                               ("count", 5, "count must be in"), ("xs", 17, "4-byte aligned")):
        bad = (_native.ChainLaunch * 1)()
        ctypes.pointer(bad[0])[0] = one[0]
        setattr(bad[0], field, value)
        assert lib.mambo_iq3s_fp8_matmul_chain(1, bad, 1, None, sp, None) == _native.MAMBO_ERR_VALUE, field
        assert text in lib.mambo_last_error().decode(), (field, lib.mambo_last_error())
    cfg = _native.ChainConfig()
    cfg.waves = 6
    assert lib.mambo_iq3s_fp8_matmul_chain(1, one, 1, cfg, sp, None) == _native.MAMBO_ERR_VALUE
    assert "waves" in lib.mambo_last_error().decode()
    cfg.waves, cfg.tiles_per_workgroup = 4, -1
    assert lib.mambo_iq3s_fp8_matmul_chain(1, one, 1, cfg, sp, None) == _native.MAMBO_ERR_VALUE
    assert "tiles per workgroup" in lib.mambo_last_error().decode()
