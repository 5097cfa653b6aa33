"""ctypes bindings for the CPU oracle in ``mambo_oracle.c``.

Test infrastructure only: tests/, ``__graft_entry__.smoke()`` and the
cpu_baseline leg of bench.py use it, to check results or as the timed CPU
baseline. The product package
(``mambo_amd``) never imports it.
"""

from __future__ import annotations

import ctypes
import io
import json
import math
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def _declare(L: ctypes.CDLL) -> None:
    vp, i64, u64, f64, u8, u16 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64,
                                  ctypes.c_double, ctypes.c_uint8, ctypes.c_uint16)
    L.orc_iq3s_grid.argtypes = [vp]
    L.orc_e4m3_decode.argtypes = [u8]
    L.orc_e4m3_decode.restype = ctypes.c_float
    L.orc_e4m3_encode.argtypes = [f64]
    L.orc_e4m3_encode.restype = u8
    L.orc_mxfp8_exponent.argtypes = [ctypes.c_float]
    L.orc_mxfp8_exponent.restype = ctypes.c_int
    L.orc_fp16_to_f32.argtypes = [u16]
    L.orc_fp16_to_f32.restype = ctypes.c_float
    L.orc_f32_to_fp16.argtypes = [ctypes.c_float]
    L.orc_f32_to_fp16.restype = u16
    L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    L.orc_f32_to_bf16.restype = u16
    L.orc_quantize_mxfp8_f32.argtypes = [vp, i64, i64, i64, vp, vp]
    L.orc_quantize_mxfp8_bf16.argtypes = [vp, i64, i64, i64, vp, vp]
    L.orc_mxfp8_decode.argtypes = [vp, vp, i64, i64, vp]
    L.orc_dequant_iq3s.argtypes = [vp, i64, i64, vp]
    L.orc_dequant_iq3s_fp8.argtypes = [vp, i64, i64, vp, vp]
    L.orc_matmul_f64.argtypes = [vp, i64, i64, vp, i64, vp]
    L.orc_iq3s_fp8_matmul.argtypes = [vp, i64, vp, i64, i64, vp, i64, i64, i64, i64, vp, ctypes.c_int]
    L.orc_rnd.argtypes = [u64, u64, u64]
    L.orc_rnd.restype = u64
    L.orc_normal.argtypes = [u64, u64, u64]
    L.orc_normal.restype = f64
    L.orc_gen_iq3s.argtypes = [u64, i64, i64, i64, vp]
    L.orc_gen_bf16.argtypes = [u64, u64, f64, i64, i64, vp]
    L.orc_e4m3_encode_array.argtypes = [vp, i64, vp]
    L.orc_mxfp8_exponent_array.argtypes = [vp, i64, vp]


def iq3s_grid() -> np.ndarray:
    out = np.zeros(512, dtype=np.uint32)
    lib().orc_iq3s_grid(_p(out))
    return out


def e4m3_decode_all() -> np.ndarray:
    return np.array([lib().orc_e4m3_decode(b) for b in range(256)], dtype=np.float32)


def e4m3_encode(values) -> np.ndarray:
    """Round to E4M3 (nearest even, saturating); values are taken as float64."""
    v = np.ascontiguousarray(np.asarray(values, dtype=np.float64).ravel())
    out = np.empty(v.size, dtype=np.uint8)
    lib().orc_e4m3_encode_array(_p(v), v.size, _p(out))
    return out


def mxfp8_exponent(amax) -> np.ndarray:
    """Block exponent e for each f32 amax."""
    a = np.ascontiguousarray(np.asarray(amax, dtype=np.float32).ravel())
    out = np.empty(a.size, dtype=np.int32)
    lib().orc_mxfp8_exponent_array(_p(a), a.size, _p(out))
    return out


def quantize_mxfp8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x f32 or bf16-as-uint16 [M, K] -> (E4M3 u8 [M, K], E8M0 u8 [M, K/32])."""
    x = np.ascontiguousarray(x)
    m, k = x.shape
    if k % 32:
        raise ValueError("K must be divisible by 32")
    values = np.empty((m, k), dtype=np.uint8)
    scales = np.empty((m, k // 32), dtype=np.uint8)
    if x.dtype == np.float32:
        lib().orc_quantize_mxfp8_f32(_p(x), m, k, k, _p(values), _p(scales))
    elif x.dtype == np.uint16:
        lib().orc_quantize_mxfp8_bf16(_p(x), m, k, k, _p(values), _p(scales))
    else:
        raise TypeError("x must be float32 or bfloat16 bits (uint16)")
    return values, scales


def mxfp8_decode(values: np.ndarray, scales: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    m, k = values.shape
    out = np.empty((m, k), dtype=np.float32)
    lib().orc_mxfp8_decode(_p(values), _p(scales), m, k, _p(out))
    return out


def dequant_iq3s(raw: np.ndarray) -> np.ndarray:
    """raw u8 [N, B, 110] -> f32 [N, B*256] (dequantize_row_iq3_s)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n, nb, _ = raw.shape
    out = np.empty((n, nb * 256), dtype=np.float32)
    lib().orc_dequant_iq3s(_p(raw), n, nb, _p(out))
    return out


def dequant_iq3s_fp8(raw: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """raw u8 [N, B, 110] -> (E4M3 u8 [N, B*256], f32 group scales [N, B*8])."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n, nb, _ = raw.shape
    values = np.empty((n, nb * 256), dtype=np.uint8)
    scales = np.empty((n, nb * 8), dtype=np.float32)
    lib().orc_dequant_iq3s_fp8(_p(raw), n, nb, _p(values), _p(scales))
    return values, scales


def matmul_f64(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_f64(_p(x), m, k, _p(w), n, _p(out))
    return out


def iq3s_fp8_matmul(xv: np.ndarray, xs: np.ndarray, raw: np.ndarray, *, rows: tuple[int, int] | None = None,
                    threads: int = 0) -> np.ndarray:
    """Reference CPU projection: out[M, N] over weight rows ``rows`` (default all)."""
    xv = np.ascontiguousarray(xv, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.uint8)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    m = xv.shape[0]
    n, nb, _ = raw.shape
    r0, r1 = rows if rows is not None else (0, n)
    out = np.zeros((m, n), dtype=np.float32)
    lib().orc_iq3s_fp8_matmul(_p(xv), xv.shape[1], _p(xs), xs.shape[1], m, _p(raw), n, nb, r0, r1,
                              _p(out), int(threads))
    return out


def gen_iq3s(seed: int, n_rows: int, blocks: int, row0: int = 0) -> np.ndarray:
    """Counter-based random IQ3_S blocks, rows [row0, row0+n_rows) -> u8 [n_rows, blocks, 110]."""
    raw = np.empty((n_rows, blocks, 110), dtype=np.uint8)
    lib().orc_gen_iq3s(seed, blocks, row0, n_rows, _p(raw))
    return raw


def gen_bf16(seed: int, count: int, *, outlier_seed: int = 2, outlier_frac: float = 0.0,
             start: int = 0) -> np.ndarray:
    """Counter-based bf16 ~N(0,1) (Irwin-Hall) with optional x100 outliers -> uint16 bits."""
    out = np.empty(count, dtype=np.uint16)
    lib().orc_gen_bf16(seed, outlier_seed, float(outlier_frac), start, count, _p(out))
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def default_threads() -> int:
    return len(os.sched_getaffinity(0))


# ------------------------------------------------------------------ command-line tool
CLI_PATH = HERE / "mambo_oracle_cli"
CLI_ARRAYS = ("dequant_rows", "ggml_dequant_f64", "mxfp8_f64")


def read_cli_packet(packet: bytes, *, m: int, k: int, n: int, rows: int) -> tuple[dict, dict]:
    """Parse mambo_oracle_cli's stdout: a u8 .npy array of JSON metadata, then the three
    float32 arrays it lists, nothing after them (the checks of the reference harness,
    compute_reference_gguf.py:124-151)."""
    stream = io.BytesIO(packet)
    meta = np.load(stream, allow_pickle=False)
    if meta.dtype != np.uint8 or meta.ndim != 1 or not 0 < meta.size <= 1 << 16:
        raise ValueError("oracle CLI stdout has invalid NumPy metadata")
    header = json.loads(meta.tobytes().decode("utf-8"))
    if header.get("schema_version") != 1 or header.get("op") != "matmul":
        raise ValueError("oracle CLI stdout uses an unsupported schema or op")
    shapes = {"dequant_rows": [rows, k], "ggml_dequant_f64": [m, n], "mxfp8_f64": [m, n]}
    if [d.get("name") for d in header.get("arrays", [])] != list(CLI_ARRAYS):
        raise ValueError("oracle CLI stdout has an unexpected array table")
    arrays = {}
    for d in header["arrays"]:
        name, shape = d["name"], shapes[d["name"]]
        a = np.load(stream, allow_pickle=False)
        if d.get("dtype") != "float32" or d.get("shape") != shape or d.get("nbytes") != 4 * math.prod(shape):
            raise ValueError(f"oracle CLI stdout has invalid metadata for {name}")
        if a.dtype != np.dtype("<f4") or list(a.shape) != shape or not a.flags.c_contiguous:
            raise ValueError(f"oracle CLI stdout has an invalid NumPy array for {name}")
        arrays[name] = a
    if stream.read(1):
        raise ValueError("oracle CLI stdout has trailing bytes")
    return arrays, header


def cli_matmul(model, weight: str, x: np.ndarray, *, dequant_rows: int = 4) -> tuple[dict, dict]:
    """Run mambo_oracle_cli on float32 activations x [M, K] and parse its arrays."""
    x = np.ascontiguousarray(x, dtype="<f4")
    if not CLI_PATH.exists():
        build()
    run = subprocess.run([str(CLI_PATH), "--op", "matmul", "--model", str(model), "--weight", weight,
                          "--m", str(x.shape[0]), "--dequant-rows", str(dequant_rows)],
                         input=x.tobytes(), capture_output=True, check=False)
    if run.returncode != 0:
        raise RuntimeError(f"oracle CLI failed: {run.stderr.decode(errors='replace').strip()}")
    meta = np.load(io.BytesIO(run.stdout), allow_pickle=False)
    k, n = json.loads(meta.tobytes().decode())["shape_ggml_ne_order"]
    return read_cli_packet(run.stdout, m=x.shape[0], k=k, n=n, rows=dequant_rows)
