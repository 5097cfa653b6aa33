"""Shared test configuration.

Markers: ``gpu`` tests need an MI355X (gfx950) and call the HIP library through the
C ABI; everything else runs on the CPU (oracle pins, ABI exports, host logic).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
GOLDEN = Path(__file__).resolve().parent / "golden"
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU; runs the HIP kernels through the C ABI")


@pytest.fixture(scope="session")
def gpu():
    """The current torch device. GPU tests fail (not skip) if the HIP library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from mambo_amd import _native
    _native.lib()  # raises if libmambo_hip.so was not built
    arch = _native.device_arch()
    if arch != "gfx950":
        pytest.skip(f"device is {arch}, kernels are built for gfx950")
    return torch.device("cuda", torch.cuda.current_device())


def make_synthetic_iq3_s(n_rows: int, k: int, seed: int) -> np.ndarray:
    """Random IQ3_S blocks as the reference test builds them (test_iq3_s_fp8.py:41-51):
    all bytes uniform, then d ~ U(0.002, 0.04) as fp16."""
    if k % 256:
        raise ValueError("IQ3_S synthetic K must be divisible by 256")
    blocks = k // 256
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(n_rows, blocks, 110), dtype=np.uint8)
    base_scales = rng.uniform(0.002, 0.04, size=(n_rows, blocks)).astype("<f2")
    raw[..., :2] = base_scales.view(np.uint8).reshape(n_rows, blocks, 2)
    return raw


def all_codes_blocks() -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Every codebook index with every sign nibble (test_iq3_s_fp8.py:108-117):
    8 rows x 16 blocks = 8192 four-weight codes, d = 1, scale nibbles 0.
    Returns (raw [8,16,110], code index per code [8,16,64], sign nibble per code)."""
    n_rows, blocks = 8, 16
    raw = np.zeros((n_rows, blocks, 110), dtype=np.uint8)
    raw[..., :2] = np.array([1.0], dtype=np.float16).view(np.uint8)
    code = (np.arange(8192, dtype=np.uint16) % 512).reshape(n_rows, blocks, 64)
    sign = (np.arange(8192, dtype=np.uint16) // 512).reshape(n_rows, blocks, 64)
    raw[..., 2:66] = code.astype(np.uint8)
    raw[..., 66:74] = np.packbits((code >> 8).astype(np.uint8), axis=-1, bitorder="little")
    raw[..., 74:106] = (sign[..., 0::2] | (sign[..., 1::2] << 4)).astype(np.uint8)
    return raw, code, sign


# ---------------------------------------------------------------- independent codecs
# Written from the OCP FP8 definition (E4M3, bias 7, S.1111.111 = NaN), independent of
# the C oracle; fp8_reference.py:10-43 in the reference holds the same closed form.
def e4m3_values() -> np.ndarray:
    codes = np.arange(256, dtype=np.uint16)
    e = (codes >> 3) & 15
    m = (codes & 7).astype(np.float64)
    v = np.where(e == 0, m * 2.0**-9, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(codes & 0x80, -v, v)


def e4m3_encode_bruteforce(x: np.ndarray) -> np.ndarray:
    """Nearest finite E4M3 code by exhaustive distance, ties to the even code,
    saturating; sign from the input (including -0)."""
    x = np.asarray(x, dtype=np.float64).ravel()
    pos = e4m3_values()[:127]  # codes 0..126: 0 and the 126 finite positive values
    # beyond 2*448 every distance comparison is decided by saturation; clamping keeps
    # the float64 distances exact
    a = np.minimum(np.abs(x), 1024.0)
    out = np.empty(x.size, dtype=np.uint8)
    for start in range(0, x.size, 1 << 16):
        aa = a[start:start + (1 << 16)]
        dist = np.abs(aa[:, None] - pos[None, :])
        best = dist.min(axis=1, keepdims=True)
        cand = dist == best
        # among equidistant codes prefer the even one
        even = cand & ((np.arange(127) & 1) == 0)[None, :]
        pick = np.where(even.any(axis=1), even.argmax(axis=1), cand.argmax(axis=1))
        out[start:start + aa.size] = pick
    return out | np.where(np.signbit(x), 0x80, 0).astype(np.uint8)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.sqrt(np.sum(b * b))
    return float(np.sqrt(np.sum((a - b) ** 2)) / (den if den > 0 else 1.0))
