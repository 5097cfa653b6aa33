"""ctypes binding of libmambo_hip.so (the C ABI declared in include/mambo_hip.h).

The library holds the gfx950 kernels; this module only loads it, declares the entry
points and maps status codes to the Python exceptions the reference launchers raise
(ValueError / TypeError / RuntimeError). There is no fallback: if the library is
missing, every operator raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmambo_hip.so"

MAMBO_OK = 0
MAMBO_ERR_VALUE = -1
MAMBO_ERR_TYPE = -2
MAMBO_ERR_RUNTIME = -3
MAMBO_ERR_UNSUPPORTED = -4

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_MXFP8 = 2

GEMM_AUTO = 0
GEMM_STREAM = 1
GEMM_TILED = 2
GEMM_DENSE = 3


class GemmConfig(ctypes.Structure):
    """mirror of mambo_gemm_config"""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("split_k", ctypes.c_int32),
        ("tile_m", ctypes.c_int32),
        ("tile_n", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 3),
    ]

    def as_dict(self) -> dict:
        return {"kernel": self.kernel, "waves": self.waves, "split_k": self.split_k,
                "tile_m": self.tile_m, "tile_n": self.tile_n}

    @classmethod
    def from_dict(cls, d: dict) -> "GemmConfig":
        c = cls()
        c.kernel = int(d.get("kernel", GEMM_STREAM))
        c.waves = int(d.get("waves", 0))
        c.split_k = int(d.get("split_k", 0))
        c.tile_m = int(d.get("tile_m", 0))
        c.tile_n = int(d.get("tile_n", 0))
        return c


MAX_GROUP = 4


class Projection(ctypes.Structure):
    """mirror of mambo_projection"""

    _fields_ = [("packed", ctypes.c_void_p), ("n", ctypes.c_int64), ("out", ctypes.c_void_p), ("ldo", ctypes.c_int64)]


MAX_CHAIN = 16  # MAMBO_MAX_CHAIN
CHAIN_SYNC_WORDS = 4224  # MAMBO_CHAIN_SYNC_WORDS
NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024  # MAMBO_NOALLOC_SCRATCH_BYTES


class ChainLaunch(ctypes.Structure):
    """mirror of mambo_chain_launch"""

    _fields_ = [("x", ctypes.c_void_p), ("x_dtype", ctypes.c_int32), ("count", ctypes.c_int32),
                ("ldx", ctypes.c_int64), ("xs", ctypes.c_void_p), ("ldxs", ctypes.c_int64),
                ("blocks", ctypes.c_int64), ("proj", Projection * MAX_GROUP)]


class ChainConfig(ctypes.Structure):
    """mirror of mambo_chain_config"""

    _fields_ = [("waves", ctypes.c_int32), ("tiles_per_workgroup", ctypes.c_int32), ("timeout_us", ctypes.c_int64),
                ("wait_bias", ctypes.c_int32), ("reserved", ctypes.c_int32 * 3)]


# name -> (restype, argtypes); every symbol here is declared in include/mambo_hip.h.
_vp, _i64, _i32, _u64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint64
SIGNATURES = {
    "mambo_last_error": (ctypes.c_char_p, []),
    "mambo_abi_version": (_i32, []),
    "mambo_build_arch": (ctypes.c_char_p, []),
    "mambo_device_arch": (_i32, [_i32, ctypes.c_char_p, _i32]),
    "mambo_iq3s_grid": (_i32, [_vp]),
    "mambo_iq3s_fp8_grid": (_i32, [_vp]),
    "mambo_iq3s_split_table": (_i32, [_vp]),
    "mambo_quantize_mxfp8": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "mambo_iq3s_packed_bytes": (_i64, [_i64, _i64]),
    "mambo_iq3s_prepare": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mambo_iq3s_pack": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp]),
    "mambo_iq3s_dequant": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "mambo_iq3s_fp8_matmul": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                     ctypes.POINTER(GemmConfig), _vp]),
    "mambo_iq3s_fp8_matmul_grouped": (_i32, [_vp, _i64, _vp, _i64, _i64, ctypes.POINTER(Projection), _i32, _i64,
                                             ctypes.POINTER(GemmConfig), _vp]),
    "mambo_iq3s_matmul_quantize_grouped": (_i32, [_vp, _i32, _i64, _i64, ctypes.POINTER(Projection), _i32, _i64,
                                                  ctypes.POINTER(GemmConfig), _vp, _i64, _vp, _i64, _vp]),
    "mambo_iq3s_matmul_quantize_grouped_noalloc": (_i32, [_vp, _i32, _i64, _i64, ctypes.POINTER(Projection), _i32,
                                                          _i64, ctypes.POINTER(GemmConfig), _vp]),
    "mambo_iq3s_fp8_matmul_chain": (_i32, [_i64, ctypes.POINTER(ChainLaunch), _i32, ctypes.POINTER(ChainConfig),
                                           _vp, _vp]),
    "mambo_chain_status": (_i32, [_vp]),
    "mambo_gemm_default_config": (_i32, [_i64, _i64, _i64, ctypes.POINTER(GemmConfig)]),
    "mambo_gemm_check_config": (_i32, [_i64, _i64, _i64, ctypes.POINTER(GemmConfig)]),
    "mambo_gemm_config_enumerate": (_i64, [_i64, _i64, _i64, ctypes.POINTER(GemmConfig), _i64]),
    "mambo_synth_iq3s": (_i32, [_u64, _i64, _i64, _i64, _vp, _vp]),
    "mambo_synth_bf16": (_i32, [_u64, _u64, ctypes.c_double, _i64, _i64, _vp, _vp]),
    "mambo_e4m3_convert": (_i32, [_vp, _i64, _vp, _vp, _vp]),
    "mambo_fill_f32": (_i32, [_vp, _i64, ctypes.c_float, _vp]),
    "mambo_copy_bytes": (_i32, [_vp, _vp, _i64, _vp]),
    "mambo_read_bytes": (_i32, [_vp, _i64, _vp, _vp]),
    "mambo_mfma_peak": (_i32, [_i64, ctypes.c_int, _vp, _vp]),
}

READ_SINK_WORDS = 2048 * 256  # MAMBO_READ_SINK_WORDS

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libmambo_hip.so once; raise RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m mambo_amd.csrc.build` "
                    "(there is no non-HIP fallback)")
            handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | ctypes.RTLD_GLOBAL)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc == MAMBO_OK:
        return
    msg = lib().mambo_last_error().decode(errors="replace")
    text = f"{what}: {msg}" if what else msg
    if rc == MAMBO_ERR_VALUE:
        raise ValueError(text)
    if rc == MAMBO_ERR_TYPE:
        raise TypeError(text)
    raise RuntimeError(text)


def stream_handle(stream) -> int:
    """HIP stream handle of `stream` (None = torch's current stream on the current device)."""
    if stream is None:
        import torch
        return int(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return stream
    handle = getattr(stream, "cuda_stream", None)
    if handle is None:
        handle = getattr(stream, "ptr", None)
    if handle is None:
        raise TypeError("stream must be None, an int handle or a torch.cuda.Stream")
    return int(handle)


def device_arch(device=None) -> str:
    """gfx name of the current (or given) torch device, e.g. 'gfx950'."""
    import torch
    props = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
    return str(getattr(props, "gcnArchName", "")).split(":")[0]


def ptr(t) -> int:
    return int(t.data_ptr())
