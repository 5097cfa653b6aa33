"""Runtime ABI manifests of libmambo_hip.so (schema version 1).

One JSON document per ``extern "C"`` entry point of ``include/mambo_hip.h``, written
next to the library (``mambo_amd/abi/<symbol>.abi.json``) so a C or C++ consumer can
check, before it calls anything, that the library it loads has the ABI it was built
against. This is the counterpart of the reference's AOT export metadata
(``src/python/mambo/utils/cutile_to_cubin.py:158-177``: ``schema_version`` 1,
``name == symbol``, ordered ``parameters`` of ``{name, type}``, per-array
``constraints``, ``toolchain``; compile-time constants omitted). The reference
describes one cubin kernel whose arrays expand to ``(ptr, shape..., stride...)``; here
the unit is a host entry point of the C ABI (the library computes grids itself), so
``library_path`` replaces ``cubin_path`` and there is no launch grid.

The parameter list is parsed from the header, so it cannot drift from the
declarations; ``CONSTRAINTS`` adds, for every pointer parameter, what the header states
in prose: element type, shape and strides in terms of the other parameters, alignment,
host or device memory, whether NULL is allowed and whether it is read or written.

    python -m mambo_amd.abi [out_dir]     # writes the manifests (build() does this)
"""

from __future__ import annotations

import json
import platform
import re
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
HEADER = REPO / "include" / "mambo_hip.h"
LIBRARY = PKG / "libmambo_hip.so"
ABI_DIR = PKG / "abi"

SCHEMA_VERSION = 1
CALLING_CONVENTION = "mambo_c_abi_v1"
GPU_CODE = "gfx950"
ABI_VERSION = 100  # mambo_abi_version()

# C spellings in the header -> ABI type names (the vocabulary the C++ loader derives
# from the compiled declarations: mambo_amd/csrc/loadtest.cpp).
_SCALARS = {
    "void": "void", "char": "char", "int": "int32", "int32_t": "int32", "int64_t": "int64",
    "uint8_t": "uint8", "uint16_t": "uint16", "uint32_t": "uint32", "uint64_t": "uint64",
    "float": "float32", "double": "float64", "mambo_gemm_config": "mambo_gemm_config",
    "mambo_projection": "mambo_projection", "mambo_stream_t": "hipStream_t",
    "mambo_chain_launch": "mambo_chain_launch", "mambo_chain_config": "mambo_chain_config",
}


def _abi_type(spelling: str) -> str:
    spelling = " ".join(spelling.replace("*", " * ").split())
    const = spelling.startswith("const ")
    if const:
        spelling = spelling[len("const "):]
    stars = spelling.count("*")
    base = spelling.replace("*", "").strip()
    if base not in _SCALARS:
        raise ValueError(f"type {base!r} has no ABI name")
    return ("const " if const else "") + _SCALARS[base] + "*" * stars


def parse_header(path: Path = HEADER) -> list[dict]:
    """[{symbol, returns, parameters: [{name, type}]}] for every function the header
    declares, in declaration order."""
    text = path.read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    text = re.sub(r"^\s*#[^\n]*", " ", text, flags=re.M)
    out = []
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(mambo_\w+)\s*\(([^()]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        ret = ret.split("}")[-1].split(";")[-1].strip()
        plist = []
        if params and params != "void":
            for p in params.split(","):
                pm = re.fullmatch(r"\s*(.*?[\s\*])(\w+)\s*", p)
                if pm is None:
                    raise ValueError(f"cannot parse parameter {p!r} of {name}")
                plist.append({"name": pm.group(2), "type": _abi_type(pm.group(1))})
        out.append({"symbol": name, "returns": _abi_type(ret), "parameters": plist})
    return out


def _arr(name, dtype, shape, strides=None, *, align=1, memory="device", nullable=False, access="read"):
    shape = [str(s) for s in shape]
    return {"name": name, "kind": "array", "dtype": dtype, "ndim": len(shape), "shape": shape,
            "strides": [str(s) for s in (strides if strides is not None else _contiguous(shape))],
            "base_addr_divisible_by": align, "memory": memory, "nullable": nullable, "access": access}


def _contiguous(shape):
    strides, acc = [], "1"
    for s in reversed(shape):
        strides.append(acc)
        acc = s if acc == "1" else f"({s})*{acc}"
    return list(reversed(strides))


_PACKED = "mambo_iq3s_packed_bytes(n, blocks)"
_FIELDS_IN = [
    _arr("d", "uint16", ["blocks", "n"]), _arr("qs", "uint32", ["blocks", "n", "16"], align=4),
    _arr("qh", "uint16", ["blocks", "n", "4"], align=2), _arr("signs", "int32", ["blocks", "n", "8"], align=4),
    _arr("scales", "uint32", ["blocks", "n"], align=4),
]


def _fields_out(nullable: bool):
    return [dict(c, nullable=nullable, access="write") for c in _FIELDS_IN]


# Every pointer parameter of every entry point: what the header's prose states.
CONSTRAINTS: dict[str, list[dict]] = {
    "mambo_last_error": [],
    "mambo_abi_version": [],
    "mambo_build_arch": [],
    "mambo_device_arch": [_arr("buf", "char", ["buf_len"], memory="host", access="write")],
    "mambo_iq3s_grid": [_arr("out", "uint32", ["512"], align=4, memory="host", access="write")],
    "mambo_iq3s_fp8_grid": [_arr("out", "uint32", ["512"], align=4, memory="host", access="write")],
    "mambo_iq3s_split_table": [_arr("out", "uint32", ["64"], align=4, memory="host", access="write")],
    "mambo_quantize_mxfp8": [
        _arr("x", "float32|bfloat16", ["m", "k"], ["ldx", "1"], align=2),
        _arr("values", "uint8", ["m", "k"], ["ldv", "1"], access="write"),
        _arr("scales", "uint8", ["m", "k/32"], ["lds", "1"], access="write"),
    ],
    "mambo_iq3s_packed_bytes": [],
    "mambo_iq3s_prepare": [
        _arr("raw", "uint8", ["n", "blocks", "110"], ["stride_n", "stride_b", "stride_byte"]),
        *_fields_out(True),
        _arr("packed", "uint8", [_PACKED], align=16, nullable=True, access="write"),
    ],
    "mambo_iq3s_pack": [*_FIELDS_IN, _arr("packed", "uint8", [_PACKED], align=16, access="write")],
    "mambo_iq3s_dequant": [
        *_FIELDS_IN,
        _arr("values", "uint8", ["n", "blocks*256"], access="write"),
        _arr("out_scales", "float32", ["n", "blocks*8"], align=4, access="write"),
    ],
    "mambo_iq3s_fp8_matmul": [
        _arr("xv", "uint8", ["m", "blocks*256"], ["ldxv", "1"], align=16),
        _arr("xs", "uint8", ["m", "blocks*8"], ["ldxs", "1"]),
        _arr("packed", "uint8", [_PACKED], align=16),
        _arr("out", "float32", ["m", "n"], ["ldo", "1"], align=4, access="write"),
        _arr("cfg", "mambo_gemm_config", ["1"], align=4, memory="host", nullable=True),
    ],
    "mambo_iq3s_fp8_matmul_grouped": [
        _arr("xv", "uint8", ["m", "blocks*256"], ["ldxv", "1"], align=16),
        _arr("xs", "uint8", ["m", "blocks*8"], ["ldxs", "1"]),
        _arr("proj", "mambo_projection", ["count"], align=8, memory="host"),
        _arr("cfg", "mambo_gemm_config", ["1"], align=4, memory="host", nullable=True),
    ],
    "mambo_iq3s_matmul_quantize_grouped": [
        _arr("x", "float32|bfloat16", ["m", "blocks*256"], ["ldx", "1"], align=2),
        _arr("proj", "mambo_projection", ["count"], align=8, memory="host"),
        _arr("cfg", "mambo_gemm_config", ["1"], align=4, memory="host", nullable=True),
        _arr("xv", "uint8", ["m", "blocks*256"], ["ldxv", "1"], align=16, access="write"),
        _arr("xs", "uint8", ["m", "blocks*8"], ["ldxs", "1"], access="write"),
    ],
    "mambo_iq3s_matmul_quantize_grouped_noalloc": [
        _arr("x", "float32|bfloat16", ["m", "blocks*256"], ["ldx", "1"], align=2),
        _arr("proj", "mambo_projection", ["count"], align=8, memory="host"),
        _arr("cfg", "mambo_gemm_config", ["1"], align=4, memory="host", nullable=True),
    ],
    "mambo_iq3s_fp8_matmul_chain": [
        _arr("launches", "mambo_chain_launch", ["count"], align=8, memory="host"),
        _arr("cfg", "mambo_chain_config", ["1"], align=8, memory="host", nullable=True),
        _arr("sync", "uint32", ["MAMBO_CHAIN_SYNC_WORDS"], align=4, access="readwrite"),
    ],
    "mambo_chain_status": [_arr("sync", "uint32", ["MAMBO_CHAIN_SYNC_WORDS"], align=4, access="readwrite")],
    "mambo_gemm_default_config": [_arr("out", "mambo_gemm_config", ["1"], align=4, memory="host", access="write")],
    "mambo_gemm_check_config": [_arr("cfg", "mambo_gemm_config", ["1"], align=4, memory="host")],
    "mambo_gemm_config_enumerate": [
        _arr("out", "mambo_gemm_config", ["capacity"], align=4, memory="host", nullable=True, access="write")],
    "mambo_synth_iq3s": [_arr("raw", "uint8", ["nrows", "blocks", "110"], access="write")],
    "mambo_synth_bf16": [_arr("out", "uint16", ["count"], align=2, access="write")],
    "mambo_e4m3_convert": [
        _arr("in", "float32", ["n"], align=4),
        _arr("out_sw", "uint8", ["n"], nullable=True, access="write"),
        _arr("out_hw", "uint8", ["n"], nullable=True, access="write"),
    ],
    "mambo_fill_f32": [_arr("ptr", "float32", ["n"], align=4, access="write")],
    "mambo_copy_bytes": [_arr("src", "uint8", ["bytes"], align=16), _arr("dst", "uint8", ["bytes"], align=16,
                                                                         access="write")],
    "mambo_read_bytes": [_arr("src", "uint8", ["bytes"], align=16),
                         _arr("sink", "uint32", ["MAMBO_READ_SINK_WORDS"], align=4, access="write")],
    "mambo_mfma_peak": [_arr("out", "float32", ["workgroups*256"], align=4, access="write")],
}


def _hipcc_version() -> str:
    for cand in ("/opt/rocm/bin/hipcc", "hipcc"):
        try:
            proc = subprocess.run([cand, "--version"], capture_output=True, text=True, timeout=60)
        except (OSError, subprocess.SubprocessError):
            continue
        for line in proc.stdout.splitlines():
            if line.startswith("HIP version"):
                return line.split(":", 1)[1].strip()
    return "unknown"


def manifests(library_path: str = "../libmambo_hip.so", toolchain: dict | None = None) -> list[dict]:
    """The manifest documents, one per declared entry point. ``library_path`` is
    resolved by the loader relative to the manifest's directory when not absolute."""
    toolchain = toolchain or {"python": platform.python_version(), "hipcc": _hipcc_version()}
    docs = []
    for fn in parse_header():
        sym = fn["symbol"]
        if sym not in CONSTRAINTS:
            raise ValueError(f"{sym} is declared in {HEADER.name} but has no constraint entry")
        pointers = {p["name"] for p in fn["parameters"] if p["type"].endswith("*")}
        named = [c["name"] for c in CONSTRAINTS[sym]]
        if sorted(named) != sorted(pointers):
            raise ValueError(f"{sym}: constraints {named} do not cover the pointer parameters {sorted(pointers)}")
        docs.append({
            "schema_version": SCHEMA_VERSION,
            "name": sym,
            "symbol": sym,
            "library_path": library_path,
            "gpu_code": GPU_CODE,
            "calling_convention": CALLING_CONVENTION,
            "abi_version": ABI_VERSION,
            "returns": fn["returns"],
            "parameters": fn["parameters"],
            "constraints": CONSTRAINTS[sym],
            "toolchain": toolchain,
        })
    return docs


def write_manifests(out_dir: Path = ABI_DIR, library_path: str | None = None) -> list[Path]:
    """Write ``<symbol>.abi.json`` for every entry point into out_dir, and remove the
    manifests of symbols the library no longer exports."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    if library_path is None:
        library_path = str(Path("..") / LIBRARY.name) if out_dir.resolve() == ABI_DIR else str(LIBRARY)
    paths = []
    for doc in manifests(library_path):
        path = out_dir / f"{doc['symbol']}.abi.json"
        path.write_text(json.dumps(doc, indent=2, sort_keys=True) + "\n", encoding="utf-8")
        paths.append(path)
    for stale in set(out_dir.glob("*.abi.json")) - set(paths):
        stale.unlink()
    return paths


if __name__ == "__main__":
    target = Path(sys.argv[1]) if len(sys.argv) > 1 else ABI_DIR
    for p in write_manifests(target):
        print(p)
