"""Every entry of the committed tuned table (mambo_amd/kernels/tuned_gfx950.json) at its
own shape: the entry's configuration for N x K at the largest token count of its bucket
and at the smallest (M = bucket/2 + 1, ragged token tiles), sampled output rows against
the oracle (weights from the counter-based generator, which the oracle regenerates row
by row). The table is what launch_iq3_s_fp8_matmul uses by default on gfx950, so each of
its configurations is a launch path the benchmark and callers take.

Tolerance: rel-L2 <= 1e-3 against the oracle's float64-accumulated product of the
decoded operands (the path's acceptance bar)."""

from __future__ import annotations

import json

import pytest
import torch

from test_gpu_configs import columns, oracle_rows, sample_rows
from test_gpu_matmul import _synth_act, _synth_weight, check, step

pytestmark = pytest.mark.gpu


def _entries():
    from mambo_amd.kernels import iq3_s_fp8
    table = json.loads(iq3_s_fp8.TUNED_PATH.read_text()).get("gfx950", {})
    out = []
    for key, cfg in sorted(table.items()):
        shape, bucket = key.split("@")
        n, k = map(int, shape.split("x"))
        out.append(pytest.param(n, k, int(bucket), cfg, id=key))
    return out


@pytest.mark.parametrize("n,k,bucket,cfg", _entries())
def test_tuned_entry_matches_oracle(gpu, n, k, bucket, cfg):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul, select_config
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    seed = 500 + (n // 16 + k // 256 + bucket) % 400
    step(f"synth weight {n}x{k}")
    fields = _synth_weight(gpu, n, k, seed=seed)
    rows = sample_rows(n, 24, seed)
    for m in sorted({bucket, bucket // 2 + 1}):
        assert select_config(m, n, k) == cfg, "the table's entry is the default for its bucket"
        xq, xs = launch_quantize_fp8(_synth_act(gpu, m, k, seed=seed + m))
        step(f"matmul M={m} {n}x{k} config={cfg}")
        out = launch_iq3_s_fp8_matmul(xq, xs, fields, config=cfg)
        torch.cuda.synchronize()
        check(columns(out, rows), oracle_rows(xq, xs, seed, k, rows), elementwise=False)
        assert bool(torch.isfinite(out).all())
