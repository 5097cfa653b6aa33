"""Build libmambo_hip.so (gfx950) from the .hip sources in this directory.

    python -m mambo_amd.csrc.build          # or mambo_amd.csrc.build.build()

Each translation unit is compiled in parallel with hipcc into ``_build/`` and linked
into ``mambo_amd/libmambo_hip.so`` (in-tree, so it travels with the repository). The
C++ manifest loader ``mambo_amd/mambo_loadtest`` and the runtime ABI manifests
(``mambo_amd/abi/*.abi.json``, mambo_amd/abi.py) are built next to it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
REPO = PKG.parent
OUT = PKG / "libmambo_hip.so"
LOADTEST = PKG / "mambo_loadtest"
BUILD_DIR = CSRC / "_build"
ARCH = "gfx950"

SOURCES = ["api.hip", "quantize_mxfp8.hip", "iq3s_layout.hip", "iq3s_gemm.hip", "iq3s_chain.hip", "synth.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++20",
    "-munsafe-fp-atomics",
    # Keep hipcc from emitting packed FP32 instructions (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def _compile(src: str, extra: list[str]) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return obj


def build(extra_flags: list[str] | None = None, jobs: int | None = None) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    extra = list(extra_flags or [])
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, extra), SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    build_loadtest()
    from mambo_amd import abi
    abi.write_manifests()
    return OUT


def build_loadtest() -> Path:
    """The C++ manifest loader (csrc/loadtest.cpp): host code only, linked against the
    HIP runtime, zlib and libdl; it dlopens the library rather than linking it."""
    tmp = LOADTEST.with_suffix(".tmp")
    cmd = [hipcc(), "-O2", "-std=c++20", f"-I{REPO / 'include'}", str(CSRC / "loadtest.cpp"), "-o", str(tmp),
           "-lz", "-ldl"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for loadtest.cpp:\n{proc.stderr}")
    os.replace(tmp, LOADTEST)
    return LOADTEST


if __name__ == "__main__":
    path = build(sys.argv[1:])
    print(path)
