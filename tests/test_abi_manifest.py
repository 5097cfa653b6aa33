"""Runtime ABI manifests (mambo_amd/abi.py) and the C++ loader that binds the library
through them (mambo_amd/csrc/loadtest.cpp), on the CPU: every declared entry point has
a manifest; the loader's view of the compiled declarations equals the header parse;
every manifest validates and binds; and the loader rejects what the reference's loader
rejects (tests/python/test_invalid_abi.py:12-26, loadtest.cpp:201-219) plus reordered
or retyped parameters, unconstrained pointers and a library of another ABI version."""

from __future__ import annotations

import copy
import ctypes
import json
import subprocess

import pytest

from conftest import GOLDEN, REPO

LOADTEST = REPO / "mambo_amd" / "mambo_loadtest"


def loader(*args: str) -> subprocess.CompletedProcess:
    assert LOADTEST.is_file(), f"{LOADTEST} is missing: run python -m mambo_amd.csrc.build"
    return subprocess.run([str(LOADTEST), *args], capture_output=True, text=True, timeout=60)


@pytest.fixture(scope="module")
def manifests():
    from mambo_amd import abi
    return {d["symbol"]: d for d in abi.manifests(library_path=str(abi.LIBRARY))}


def write(tmp_path, doc, name="entry.abi.json"):
    path = tmp_path / name
    path.write_text(json.dumps(doc) if not isinstance(doc, str) else doc)
    return str(path)


def test_one_manifest_per_declared_entry_point(manifests):
    from mambo_amd import abi
    from test_abi import declared_symbols
    assert sorted(manifests) == declared_symbols()
    for doc in manifests.values():
        assert doc["schema_version"] == 1 and doc["name"] == doc["symbol"]
        assert doc["calling_convention"] == "mambo_c_abi_v1" and doc["gpu_code"] == "gfx950"
        assert "constants" not in doc
    assert abi.ABI_VERSION == 100


def test_writing_removes_manifests_of_symbols_no_longer_exported(tmp_path):
    from mambo_amd import abi
    stale = tmp_path / "mambo_removed_entry_point.abi.json"
    stale.write_text("{}\n")
    written = abi.write_manifests(tmp_path)
    assert not stale.exists()
    assert sorted(p.name for p in tmp_path.iterdir()) == sorted(p.name for p in written)


def test_loader_declarations_equal_the_header_parse(manifests):
    """The loader derives parameter types from the compiled declarations (decltype);
    the Python side parses the header text. Both must read the same ABI."""
    run = loader("--list")
    assert run.returncode == 0, run.stderr
    compiled = {}
    for line in run.stdout.splitlines():
        sym, ret, *params = line.split("\t")
        compiled[sym] = (ret, [dict(zip(("type", "name"), p.rsplit(":", 1))) for p in params])
    assert set(compiled) == set(manifests)
    for sym, doc in manifests.items():
        ret, params = compiled[sym]
        assert ret == doc["returns"], sym
        assert params == doc["parameters"], sym


def test_every_manifest_validates_and_binds(manifests, tmp_path):
    for sym, doc in manifests.items():
        path = write(tmp_path, doc, f"{sym}.abi.json")
        run = loader("--validate-abi-json", path)
        assert run.returncode == 0 and f"valid for entry point {sym}" in run.stdout, run.stderr
        run = loader("--abi-json", path)
        assert run.returncode == 0 and f"bound {sym}" in run.stdout, run.stderr


def test_in_tree_manifests_bind_the_in_tree_library():
    from mambo_amd import abi
    path = abi.ABI_DIR / "mambo_iq3s_fp8_matmul.abi.json"
    assert path.is_file(), "build() writes the manifests next to the library"
    run = loader("--abi-json", str(path))
    assert run.returncode == 0 and "libmambo_hip.so" in run.stdout, run.stderr


def test_rejects_unsupported_schema():
    """tests/python/test_invalid_abi.py:12-26 with the reference's fixture
    (tests/fixtures/invalid_schema.abi.json)."""
    run = loader("--validate-abi-json", str(GOLDEN / "invalid_schema.abi.json"))
    assert run.returncode != 0, "loadtest accepted unsupported ABI schema version"
    assert "schema_version 1 is required" in run.stderr, run.stderr


def _swap(doc, i, j):
    doc["parameters"][i], doc["parameters"][j] = doc["parameters"][j], doc["parameters"][i]


def _set(key, value):
    def f(doc):
        doc[key] = value
    return f


def _constraint(name, key, value):
    def f(doc):
        next(c for c in doc["constraints"] if c["name"] == name)[key] = value
    return f


MUTATIONS = [
    ("constants", _set("constants", {"tile": 4}), "compile-time constants must be omitted"),
    ("calling convention", _set("calling_convention", "cutile_python_v2"), "unsupported calling convention"),
    ("name != symbol", _set("name", "mambo_other"), "name and symbol must be matching strings"),
    ("unknown key", _set("cubin_path", "x.cubin"), "unknown=cubin_path"),
    ("missing key", lambda d: d.pop("toolchain"), "missing=toolchain"),
    ("cuda gpu code", _set("gpu_code", "sm_120"), "gpu_code must use the gfxNNN form"),
    ("abi version type", _set("abi_version", "100"), "abi_version must be a positive integer"),
    ("reordered (same types)", lambda d: _swap(d, 4, 6), "reordered ABI parameter at index 4"),
    ("retyped", lambda d: d["parameters"][1].update(type="int32"), "reordered ABI parameter at index 1"),
    ("dropped", lambda d: d["parameters"].pop(), "parameter count 11 does not match the declaration (12)"),
    ("return type", _set("returns", "int64"), "return type int64 does not match"),
    ("unconstrained pointer", lambda d: d["constraints"].pop(0), "pointer parameter xv has no constraint"),
    ("constraint on a scalar", lambda d: d["constraints"].append(dict(d["constraints"][0], name="ldxv")),
     "constraint ldxv does not name a pointer parameter"),
    ("const written", _constraint("xv", "access", "write"), "a const pointer parameter cannot be written"),
    ("alignment", _constraint("xv", "base_addr_divisible_by", 12), "power of two"),
    ("ndim vs shape", _constraint("out", "ndim", 3), "shape must list ndim extents"),
    ("dtype", _constraint("out", "dtype", "float16"), "unsupported dtype"),
    ("unknown entry point", lambda d: d.update(name="mambo_gone", symbol="mambo_gone"),
     "entry point mambo_gone is unknown to this loader"),
]


@pytest.mark.parametrize("what,mutate,message", MUTATIONS, ids=[m[0] for m in MUTATIONS])
def test_rejects_manifest_mutation(manifests, tmp_path, what, mutate, message):
    doc = copy.deepcopy(manifests["mambo_iq3s_fp8_matmul"])
    mutate(doc)
    run = loader("--validate-abi-json", write(tmp_path, doc))
    assert run.returncode == 1, f"{what}: accepted"
    assert "invalid ABI JSON" in run.stderr and message in run.stderr, run.stderr


@pytest.mark.parametrize("text,message", [
    ('{"schema_version": 1,', "malformed JSON"),
    ('{"schema_version": 1, "schema_version": 1}', "duplicate key"),
    ('[1, 2]', "root must be an object"),
    ('{"schema_version": 1.0}', "schema_version 1 is required"),
])
def test_rejects_malformed_documents(tmp_path, text, message):
    run = loader("--validate-abi-json", write(tmp_path, text))
    assert run.returncode == 1 and message in run.stderr, run.stderr


def test_binding_checks_the_library(manifests, tmp_path):
    doc = copy.deepcopy(manifests["mambo_iq3s_fp8_matmul"])
    doc["abi_version"] = 101
    run = loader("--abi-json", write(tmp_path, doc))
    assert run.returncode == 1 and "library ABI version 100 does not match the manifest's 101" in run.stderr
    doc = copy.deepcopy(manifests["mambo_iq3s_fp8_matmul"])
    doc["library_path"] = "missing/libmambo_hip.so"  # relative: resolved against the manifest's folder
    run = loader("--abi-json", write(tmp_path, doc))
    assert run.returncode == 1 and str(tmp_path / "missing" / "libmambo_hip.so") in run.stderr, run.stderr


def test_usage_errors_exit_2():
    assert loader().returncode == 2
    assert loader("--validate-abi-json").returncode == 2
    assert loader("--probe", "x.npz").returncode == 2


def test_constraint_expressions_use_only_parameters(manifests):
    """Every shape and stride expression evaluates to a positive integer from the
    entry point's own integer parameters (sample values) and the library's
    mambo_iq3s_packed_bytes / MAMBO_READ_SINK_WORDS / MAMBO_CHAIN_SYNC_WORDS."""
    from mambo_amd import _native
    lib = _native.lib()
    env = {"mambo_iq3s_packed_bytes": lambda n, b: lib.mambo_iq3s_packed_bytes(n, b),
           "MAMBO_READ_SINK_WORDS": _native.READ_SINK_WORDS, "MAMBO_CHAIN_SYNC_WORDS": _native.CHAIN_SYNC_WORDS}
    for sym, doc in manifests.items():
        ints = {p["name"]: 64 for p in doc["parameters"] if not p["type"].endswith("*")
                and p["type"] in ("int32", "int64", "uint64")}
        for c in doc["constraints"]:
            for expr in c["shape"] + c["strides"]:
                # C expressions over positive integers: '/' is integer division
                value = eval(expr.replace("/", "//"), {"__builtins__": {}}, {**env, **ints})  # noqa: S307
                assert isinstance(value, int) and value > 0, (sym, c["name"], expr)


def test_ctypes_declarations_follow_the_manifests(manifests):
    """mambo_amd/_native.py declares every entry point with argument kinds that match
    the manifest: pointers as pointers, 32/64-bit integers and floats by width."""
    from mambo_amd import _native
    kinds = {"int32": {ctypes.c_int, ctypes.c_int32}, "int64": {ctypes.c_int64}, "uint64": {ctypes.c_uint64},
             "float32": {ctypes.c_float}, "float64": {ctypes.c_double}}
    for sym, doc in manifests.items():
        restype, argtypes = _native.SIGNATURES[sym]
        assert len(argtypes) == len(doc["parameters"]), sym
        for ct, p in zip(argtypes, doc["parameters"]):
            if p["type"].endswith("*") or p["type"] == "hipStream_t":
                assert ct in (ctypes.c_void_p, ctypes.c_char_p) or issubclass(ct, ctypes._Pointer), (sym, p)
            else:
                assert ct in kinds[p["type"]], (sym, p)
