"""One GPU's shard of a tensor-parallel Llama-3 layer (the shapes `bench.py --tp G`
sweeps): at G = 2, 4, 8 the column-parallel q/k/v and gate/up keep N/G rows (k/v of the
8B model at G = 8: 128 rows) and the row-parallel o and down keep K/G columns (down of
the 8B model at G = 8: 1792 = 7 blocks, o: 512 = 2 blocks), shapes the unsharded layers
never reach. Each projection runs with the library's default configuration for its
shape at a decode, a mid and a prefill token count (stream, 16-token and 128-token
tiles), and sampled output rows are checked against the oracle.

Tolerance: rel-L2 <= 1e-3 against the oracle's float64-accumulated product of the
decoded operands (the path's acceptance bar)."""

from __future__ import annotations

import pytest
import torch

from test_gpu_configs import columns, oracle_rows, sample_rows
from test_gpu_matmul import _synth_act, _synth_weight, check, step

pytestmark = pytest.mark.gpu


def _shard_shapes():
    from mambo_amd.utils.sweep import layer_shapes
    shapes = {}
    for model in ("llama70b", "llama8b"):
        for tp in (2, 4, 8):
            for name, n, k, _ in layer_shapes(model, tp):
                shapes.setdefault((n, k), f"{model}-tp{tp}-{name}")
    return [pytest.param(n, k, id=f"{label}-{n}x{k}") for (n, k), label in sorted(shapes.items())]


@pytest.mark.parametrize("n,k", _shard_shapes())
def test_shard_projection_matches_oracle(gpu, n, k):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul, select_config
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    seed = 900 + (n // 16 + 3 * (k // 256)) % 500
    step(f"synth weight {n}x{k}")
    fields = _synth_weight(gpu, n, k, seed=seed)
    rows = sample_rows(n, 16, seed)
    for m in (1, 16, 128):
        xq, xs = launch_quantize_fp8(_synth_act(gpu, m, k, seed=seed + m))
        step(f"matmul M={m} {n}x{k} config={select_config(m, n, k)}")
        out = launch_iq3_s_fp8_matmul(xq, xs, fields)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(out).all())
        check(columns(out, rows), oracle_rows(xq, xs, seed, k, rows), elementwise=False)
