"""Write the small golden fixtures in this directory from the CPU oracle.

    python tests/golden/make_golden.py

Each .npz holds inputs and expected outputs for one case of the path; the GPU tests
compare the HIP kernels against them, and tests/test_oracle.py checks that the
oracle still reproduces them. Inputs follow the reference tests' constructions
(test_iq3_s_fp8.py:41-51, 151-175, 178-201) with numpy seeds.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

from conftest import make_synthetic_iq3_s  # noqa: E402
from oracle import oracle  # noqa: E402


def quant_rows_input(tokens: int = 5, k: int = 160, seed: int = 20261015) -> np.ndarray:
    """The reference quantizer test's rows (test_iq3_s_fp8.py:154-161)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((tokens, k)).astype(np.float32)
    x[0, :] = 0.0
    x[1, 0] = 32.0
    x[2, 32 + 7] = -64.0
    x[3, :32] *= 1.0e-4
    x[3, 32:64] = np.float32(2.0 ** -130)
    x[4, 64:96] = np.linspace(-12.0, 12.0, 32, dtype=np.float32)
    return x


def main() -> None:
    x = quant_rows_input()
    v, s = oracle.quantize_mxfp8(x)
    np.savez_compressed(HERE / "quant_rows.npz", x=x, values=v, scales=s)

    xb = oracle.gen_bf16(1, 8 * 512, outlier_seed=2, outlier_frac=0.01).reshape(8, 512)
    v, s = oracle.quantize_mxfp8(xb)
    np.savez_compressed(HERE / "quant_bf16_outliers.npz", x_bf16=xb, values=v, scales=s)

    raw = make_synthetic_iq3_s(5, 3 * 256, seed=0x1A3)
    bits, scales = oracle.dequant_iq3s_fp8(raw)
    np.savez_compressed(HERE / "decode_random.npz", raw=raw, values=bits, scales=scales,
                        weights=oracle.dequant_iq3s(raw))

    raw = make_synthetic_iq3_s(7, 768, seed=0x3F8)
    xf = np.random.default_rng(20261016).standard_normal((9, 768)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(xf)
    out = oracle.iq3s_fp8_matmul(xv, xs, raw)
    np.savez_compressed(HERE / "matmul_small.npz", raw=raw, x=xf, x_values=xv, x_scales=xs, out=out)


if __name__ == "__main__":
    main()
