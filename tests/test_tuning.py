"""Autotuner plumbing and the GGUF tensor directory on the CPU (no kernel launches).

The GGUF files are written by the test itself: a v3 header, metadata of several types
(the reader must skip them), an IQ3_S tensor in ggml ne order [K, N] and an F32 tensor,
with the data section aligned to general.alignment (kernel_benchmark.py:103-122,
gguf_manifest.py:435-545 describe the format the reference reads)."""

from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import oracle


def _gguf_string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, tensors, alignment=32, extra_meta=True, misalign=False):
    """tensors: list of (name, ne dims, ggml type id, payload bytes)."""
    meta = [("general.alignment", 4, struct.pack("<I", alignment))]
    if extra_meta:
        meta += [("general.name", 8, _gguf_string("synthetic")),
                 ("tokenizer.ggml.scores", 9, struct.pack("<IQ", 6, 3) + struct.pack("<3f", 0.5, 1.5, 2.5)),
                 ("tokenizer.ggml.tokens", 9, struct.pack("<IQ", 8, 2) + _gguf_string("a") + _gguf_string("bc")),
                 ("llama.block_count", 5, struct.pack("<i", 2))]
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for key, type_id, value in meta:
        out += _gguf_string(key) + struct.pack("<I", type_id) + value
    offsets, rel = [], 0
    for _, _, _, payload in tensors:
        offsets.append(rel + (8 if misalign else 0))
        rel += (len(payload) + alignment - 1) // alignment * alignment + alignment
    for (name, dims, type_id, _), off in zip(tensors, offsets):
        out += _gguf_string(name) + struct.pack("<I", len(dims)) + struct.pack("<" + "Q" * len(dims), *dims)
        out += struct.pack("<IQ", type_id, off)
    data_offset = (len(out) + alignment - 1) // alignment * alignment
    out += bytes(data_offset - len(out))
    blob = bytearray(rel + 64)
    for (_, _, _, payload), off in zip(tensors, offsets):
        blob[off:off + len(payload)] = payload
    path.write_bytes(bytes(out) + bytes(blob))
    return data_offset, offsets


def test_gguf_directory_of_iq3_s_tensor(tmp_path):
    from mambo_amd.utils.gguf import inspect_gguf
    n, k = 3, 512
    raw = oracle.gen_iq3s(7, n, k // 256)
    f32 = np.arange(10, dtype=np.float32)
    path = tmp_path / "m.gguf"
    data_offset, offsets = write_gguf(path, [("blk.0.ffn_up.weight", [k, n], 21, raw.tobytes()),
                                             ("output_norm.weight", [10], 0, f32.tobytes())])
    manifest = inspect_gguf(path)
    assert manifest["gguf"]["version"] == 3 and manifest["gguf"]["alignment"] == 32
    assert manifest["gguf"]["data_offset"] == data_offset
    t0, t1 = manifest["tensors"]
    assert t0["name"] == "blk.0.ffn_up.weight" and t0["shape"] == [k, n]
    assert t0["type"]["name"] == "iq3_s" and (t0["type"]["block_elements"], t0["type"]["block_bytes"]) == (256, 110)
    assert t0["row_bytes"] == 2 * 110 and t0["n_bytes"] == n * 2 * 110
    assert t0["offset"]["absolute"] == data_offset + offsets[0]
    blob = path.read_bytes()
    got = np.frombuffer(blob, dtype=np.uint8, count=t0["n_bytes"], offset=t0["offset"]["absolute"])
    np.testing.assert_array_equal(got.reshape(n, 2, 110), raw)
    assert t1["type"]["name"] == "f32" and t1["n_bytes"] == 40


def test_gguf_rejects_bad_files(tmp_path):
    from mambo_amd.utils.gguf import GGUFError, inspect_gguf
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + bytes(60))
    with pytest.raises(GGUFError, match="not a GGUF"):
        inspect_gguf(bad)
    mis = tmp_path / "mis.gguf"
    write_gguf(mis, [("w", [256, 1], 21, bytes(110))], misalign=True)
    with pytest.raises(GGUFError, match="not aligned"):
        inspect_gguf(mis)
    trunc = tmp_path / "trunc.gguf"
    write_gguf(trunc, [("w", [256, 4], 21, bytes(440))])
    trunc.write_bytes(trunc.read_bytes()[:-500])
    with pytest.raises(GGUFError, match="past the end"):
        inspect_gguf(trunc)


def test_tuned_table_round_trip_and_lookup(tmp_path, monkeypatch):
    from mambo_amd.kernels import iq3_s_fp8
    from mambo_amd.utils.kernel_benchmark import TuneResult, write_tuned_table
    path = tmp_path / "tuned.json"
    best = {"kernel": 3, "waves": 2, "split_k": 1, "tile_n": 32}
    r = TuneResult("M=16", iq3_s_fp8.tuned_key(4096, 4096, 16), best, 1.0, 1.0, 1.0, 1.0)
    write_tuned_table([r], path, "gfx950")
    other = TuneResult("M=4", iq3_s_fp8.tuned_key(4096, 4096, 4), {"kernel": 1, "waves": 4, "split_k": 1},
                       1.0, 1.0, 1.0, 1.0)
    write_tuned_table([other], path, "gfx950")  # merges into the existing table
    monkeypatch.setattr(iq3_s_fp8, "TUNED_PATH", path)
    iq3_s_fp8._tuned_table.cache_clear()
    try:
        assert iq3_s_fp8.select_config(16, 4096, 4096, arch="gfx950") == best
        assert iq3_s_fp8.select_config(13, 4096, 4096, arch="gfx950") == best  # same M bucket
        assert iq3_s_fp8.select_config(3, 4096, 4096, arch="gfx950")["waves"] == 4
        assert iq3_s_fp8.select_config(17, 4096, 4096, arch="gfx950") == iq3_s_fp8.BEST_CONFIGS["gfx950"]["medium"]
    finally:
        iq3_s_fp8._tuned_table.cache_clear()


def test_search_space_families_and_validity():
    """The library default leads every search space; stream candidates only up to 16
    tokens, dense up to 128, tiled from 5 (16-token tiles up to 64, larger ones from 32);
    every candidate passes the library's own
    configuration check for its shape (no launches)."""
    import ctypes

    from mambo_amd import _native
    from mambo_amd.kernels import iq3_s_fp8
    lib = _native.lib()
    for m, n, k in ((1, 8192, 8192), (4, 57344, 8192), (16, 4096, 14336), (32, 8192, 8192), (64, 10240, 8192),
                    (128, 4096, 4096), (512, 8192, 28672), (2048, 28672, 4096)):
        space = iq3_s_fp8.gemm_search_space(m, n, k)
        assert space[0] == iq3_s_fp8.default_config(m)
        kernels = {c["kernel"] for c in space[1:]}
        assert (_native.GEMM_STREAM in kernels) == (m <= 16), m
        assert (_native.GEMM_DENSE in kernels) == (m <= 128), m
        assert (_native.GEMM_TILED in kernels) == (m > 4), m
        assert any(c["kernel"] == _native.GEMM_TILED and c["tile_m"] == 16 for c in space) == (4 < m <= 64), m
        assert any(c["kernel"] == _native.GEMM_TILED and c["tile_m"] == 32 for c in space) == (16 < m <= 64), m
        assert len({tuple(sorted(c.items())) for c in space}) == len(space)
        for c in space:
            cfg = _native.GemmConfig.from_dict(c)
            if c["kernel"] != _native.GEMM_AUTO:
                assert lib.mambo_gemm_check_config(m, n, k // 256, ctypes.byref(cfg)) == 0, (m, n, k, c)


def test_config_enumerate_abi():
    """mambo_gemm_config_enumerate: a count query with no buffer, a truncated write that
    leaves the rest of the buffer alone, the default (all zero) first, and status codes
    for bad arguments (no launches)."""
    import ctypes

    from mambo_amd import _native
    lib = _native.lib()
    m, n, blocks = 4, 8192, 32
    count = lib.mambo_gemm_config_enumerate(m, n, blocks, None, 0)
    assert count > 1
    full = (_native.GemmConfig * count)()
    assert lib.mambo_gemm_config_enumerate(m, n, blocks, full, count) == count
    assert full[0].as_dict() == {"kernel": 0, "waves": 0, "split_k": 0, "tile_m": 0, "tile_n": 0}
    part = (_native.GemmConfig * 4)()
    for c in part:
        c.kernel = 99
    assert lib.mambo_gemm_config_enumerate(m, n, blocks, part, 3) == count
    assert [c.as_dict() for c in part[:3]] == [c.as_dict() for c in full[:3]]
    assert part[3].kernel == 99
    assert lib.mambo_gemm_config_enumerate(0, n, blocks, None, 0) == _native.MAMBO_ERR_VALUE
    assert "positive" in lib.mambo_last_error().decode()
    assert lib.mambo_gemm_config_enumerate(m, n, blocks, None, 5) == _native.MAMBO_ERR_VALUE
    assert lib.mambo_gemm_config_enumerate(m, n, blocks, ctypes.cast(part, ctypes.POINTER(_native.GemmConfig)),
                                           -1) == _native.MAMBO_ERR_VALUE


def test_tuned_table_drops_shapes_the_default_won(tmp_path, monkeypatch):
    from mambo_amd.kernels import iq3_s_fp8
    from mambo_amd.utils.kernel_benchmark import TuneResult, write_tuned_table
    path = tmp_path / "tuned.json"
    key = iq3_s_fp8.tuned_key(8192, 8192, 4)
    tuned = {"kernel": 1, "waves": 4, "split_k": 1, "tile_n": 32}
    write_tuned_table([TuneResult("M=4", key, tuned, 1.0, 1.0, 1.0, 9.0, default_us=10.0,
                                  default_of=iq3_s_fp8.default_config(4))], path, "gfx950")
    monkeypatch.setattr(iq3_s_fp8, "TUNED_PATH", path)
    iq3_s_fp8._tuned_table.cache_clear()
    try:
        assert iq3_s_fp8.select_config(4, 8192, 8192, arch="gfx950") == tuned
        won = TuneResult("M=4", key, iq3_s_fp8.default_config(4), 1.0, 1.0, 1.0, 10.0, default_us=10.0,
                         default_of=iq3_s_fp8.default_config(4))
        assert won.is_default
        write_tuned_table([won], path, "gfx950")
        iq3_s_fp8._tuned_table.cache_clear()
        assert iq3_s_fp8.select_config(4, 8192, 8192, arch="gfx950") == iq3_s_fp8.default_config(4)
    finally:
        iq3_s_fp8._tuned_table.cache_clear()


def test_committed_tuned_table_entries_are_valid():
    """Every configuration of the committed gfx950 table passes the library's own check
    for its shape (key N x K @ M bucket; no launches)."""
    import ctypes
    import json

    from mambo_amd import _native
    from mambo_amd.kernels import iq3_s_fp8
    table = json.loads(iq3_s_fp8.TUNED_PATH.read_text())["gfx950"]
    assert table
    lib = _native.lib()
    for key, cfg in table.items():
        shape, m = key.split("@")
        n, k = (int(v) for v in shape.split("x"))
        c = _native.GemmConfig.from_dict(cfg)
        assert c.kernel in (_native.GEMM_STREAM, _native.GEMM_DENSE, _native.GEMM_TILED), key
        for tokens in (int(m) // 2 + 1, int(m)):  # both ends of the bucket
            assert lib.mambo_gemm_check_config(tokens, n, k // 256, ctypes.byref(c)) == 0, (key, tokens, cfg)
