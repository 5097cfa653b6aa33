"""Minimal GGUF v2/v3 tensor-directory reader for loading IQ3_S weights.

Follows the file format as the reference's inspect_gguf reads it
(src/python/mambo/utils/gguf_manifest.py:435-545): magic "GGUF", version 2 or 3,
u64 tensor and metadata counts, typed metadata key/values (skipped here except
general.alignment), then per tensor: name, n_dims, u64 dims (ggml ne order),
u32 ggml type, u64 offset relative to the data section, which starts at the header
end rounded up to general.alignment (default 32). Only what load_gguf_weight needs
is kept: name, type (name, block elements, block bytes), shape, row/total bytes and
the absolute offset.
"""

from __future__ import annotations

import os
import struct
from pathlib import Path
from typing import Any, BinaryIO

# ggml_type id -> (name, elements per block, bytes per block) (gguf_manifest.py:30-42)
TENSOR_TYPES: dict[int, tuple[str, int, int]] = {
    0: ("f32", 1, 4), 1: ("f16", 1, 2), 2: ("q4_0", 32, 18), 3: ("q4_1", 32, 20),
    6: ("q5_0", 32, 22), 7: ("q5_1", 32, 24), 8: ("q8_0", 32, 34), 10: ("q2_k", 256, 84),
    11: ("q3_k", 256, 110), 12: ("q4_k", 256, 144), 13: ("q5_k", 256, 176), 14: ("q6_k", 256, 210),
    15: ("q8_k", 256, 292), 16: ("iq2_xxs", 256, 66), 17: ("iq2_xs", 256, 74), 18: ("iq3_xxs", 256, 98),
    19: ("iq1_s", 256, 50), 20: ("iq4_nl", 32, 18), 21: ("iq3_s", 256, 110), 22: ("iq2_s", 256, 82),
    23: ("iq4_xs", 256, 136), 24: ("i8", 1, 1), 25: ("i16", 1, 2), 26: ("i32", 1, 4), 27: ("i64", 1, 8),
    28: ("f64", 1, 8), 29: ("iq1_m", 256, 56), 30: ("bf16", 1, 2),
}

# metadata value type id -> fixed size in bytes (None: string / array)
_META_SIZES = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 8: None, 9: None, 10: 8, 11: 8, 12: 8}
_INT_FORMATS = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 10: "Q", 11: "q"}


class GGUFError(ValueError):
    """Malformed or unsupported GGUF header."""


def _read(fp: BinaryIO, n: int, what: str) -> bytes:
    data = fp.read(n)
    if len(data) != n:
        raise GGUFError(f"truncated GGUF while reading {what}")
    return data


def _u32(fp, what):
    return struct.unpack("<I", _read(fp, 4, what))[0]


def _u64(fp, what):
    return struct.unpack("<Q", _read(fp, 8, what))[0]


def _string(fp, what) -> bytes:
    n = _u64(fp, what + " length")
    if n > (1 << 30):
        raise GGUFError(f"{what} is unreasonably long ({n} bytes)")
    return _read(fp, n, what)


def _skip_value(fp, type_id: int, key: str) -> Any:
    if type_id not in _META_SIZES:
        raise GGUFError(f"metadata key {key!r} has unknown type {type_id}")
    if type_id == 8:
        _string(fp, f"metadata {key}")
        return None
    if type_id == 9:
        elem = _u32(fp, f"metadata {key} array type")
        count = _u64(fp, f"metadata {key} array length")
        if elem == 9:
            raise GGUFError(f"metadata key {key!r} contains a nested array")
        if elem == 8:
            for _ in range(count):
                _string(fp, f"metadata {key} element")
        else:
            size = _META_SIZES.get(elem)
            if size is None:
                raise GGUFError(f"metadata key {key!r} array has unknown element type {elem}")
            fp.seek(size * count, os.SEEK_CUR)
        return None
    raw = _read(fp, _META_SIZES[type_id], f"metadata {key}")
    fmt = _INT_FORMATS.get(type_id)
    return struct.unpack("<" + fmt, raw)[0] if fmt else None


def inspect_gguf(path: str | os.PathLike[str]) -> dict[str, Any]:
    """Tensor directory of a GGUF file (subset of the reference manifest schema)."""
    model_path = Path(path).expanduser().resolve()
    file_size = model_path.stat().st_size
    with model_path.open("rb") as fp:
        if _read(fp, 4, "magic") != b"GGUF":
            raise GGUFError(f"{model_path} is not a GGUF file")
        version = _u32(fp, "version")
        if version not in (2, 3):
            raise GGUFError(f"unsupported GGUF version {version}; expected 2 or 3")
        n_tensors = _u64(fp, "tensor count")
        n_meta = _u64(fp, "metadata count")
        if n_tensors > 10_000_000 or n_meta > 10_000_000:
            raise GGUFError("unreasonable GGUF header counts")
        alignment = 32
        for _ in range(n_meta):
            key = _string(fp, "metadata key").decode("utf-8", errors="replace")
            type_id = _u32(fp, f"metadata {key} type")
            value = _skip_value(fp, type_id, key)
            if key == "general.alignment":
                if not isinstance(value, int) or value <= 0 or value & (value - 1):
                    raise GGUFError("GGUF general.alignment must be a positive power of two")
                alignment = value
        headers = []
        for _ in range(n_tensors):
            name = _string(fp, "tensor name").decode("utf-8", errors="replace")
            n_dims = _u32(fp, f"tensor {name} dimension count")
            if not 1 <= n_dims <= 4:
                raise GGUFError(f"tensor {name!r} has unsupported dimension count {n_dims}")
            dims = list(struct.unpack("<" + "Q" * n_dims, _read(fp, 8 * n_dims, f"tensor {name} dims")))
            type_id = _u32(fp, f"tensor {name} type")
            rel = _u64(fp, f"tensor {name} offset")
            headers.append((name, dims, type_id, rel))
        data_offset = (fp.tell() + alignment - 1) // alignment * alignment
    tensors = []
    for name, dims, type_id, rel in headers:
        tname, block_elements, block_bytes = TENSOR_TYPES.get(type_id, (f"type{type_id}", 0, 0))
        row_bytes = n_bytes = None
        if block_elements and dims[0] % block_elements == 0:
            row_bytes = dims[0] // block_elements * block_bytes
            n_bytes = row_bytes
            for d in dims[1:]:
                n_bytes *= d
        absolute = data_offset + rel
        if rel % alignment:
            raise GGUFError(f"tensor {name!r} offset {rel} is not aligned to {alignment}")
        if n_bytes is not None and absolute + n_bytes > file_size:
            raise GGUFError(f"tensor {name!r} payload extends past the end of the file")
        tensors.append({
            "name": name, "shape": dims,
            "type": {"id": type_id, "name": tname, "block_elements": block_elements, "block_bytes": block_bytes},
            "row_bytes": row_bytes, "n_bytes": n_bytes,
            "offset": {"relative": rel, "absolute": absolute},
        })
    return {"gguf": {"version": version, "alignment": alignment, "data_offset": data_offset,
                     "tensor_count": n_tensors, "metadata_count": n_meta},
            "tensors": tensors}


def read_block_matrix(path: str | os.PathLike[str], name: str, type_name: str):
    """Bytes of the 2-D block-quantized tensor `name` as a host array u8
    [rows, row_blocks, block_bytes] (ggml ne order [K, rows]: each row is K values in
    K / block_elements blocks). ValueError if the file has no such tensor, if it is not
    a 2-D `type_name` tensor, or if its sizes disagree with its block layout."""
    import numpy as np

    directory = {t["name"]: t for t in inspect_gguf(path)["tensors"]}
    if name not in directory:
        raise ValueError(f"GGUF has no tensor named {name!r}")
    entry = directory[name]
    kind = entry["type"]
    if kind["name"] != type_name or len(entry["shape"]) != 2:
        raise ValueError(f"{name} must be a 2D {type_name} tensor")
    width, rows = entry["shape"]
    per_block, block_bytes = kind["block_elements"], kind["block_bytes"]
    row_blocks = width // per_block if per_block else 0
    layout_ok = (per_block > 0 and block_bytes > 0 and row_blocks * per_block == width
                 and entry["row_bytes"] == row_blocks * block_bytes
                 and entry["n_bytes"] == rows * entry["row_bytes"])
    if not layout_ok:
        raise ValueError(f"{name} has an inconsistent GGUF block layout")
    data = np.fromfile(path, dtype=np.uint8, count=entry["n_bytes"], offset=entry["offset"]["absolute"])
    return data.reshape(rows, row_blocks, block_bytes)
