"""Activation quantization inside the projection (mambo_iq3s_matmul_quantize_grouped /
launch_iq3_s_matmul_quantize): for M <= 4 on the stream kernel every workgroup
quantizes the rows into its LDS copy, so the result must equal, bit for bit, what
launch_quantize_fp8 followed by launch_iq3_s_fp8_matmul returns under the same config
(the same E4M3 codes and scales reach the same MFMAs); the caller's MXFP8 buffers stay
untouched there. Other shapes quantize into those buffers first. Both paths are also
checked against the oracle (rel-L2 <= 1e-3)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_l2
from oracle import oracle

pytestmark = pytest.mark.gpu


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


def weight(gpu, n: int, k: int, seed: int):
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    raw = oracle.gen_iq3s(seed, n, k // 256)
    return raw, prepare_iq3_s_fields(torch.from_numpy(raw).to(gpu))


def two_step(x, fields, config):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_fp8_matmul, launch_iq3_s_fp8_matmul_grouped
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    xv, xs = launch_quantize_fp8(x)
    if isinstance(fields, list):
        return launch_iq3_s_fp8_matmul_grouped(xv, xs, fields, config=config), (xv, xs)
    return launch_iq3_s_fp8_matmul(xv, xs, fields, config=config), (xv, xs)


CONFIGS = [None, {"kernel": 1, "waves": 1}, {"kernel": 1, "waves": 4, "tile_n": 32},
           {"kernel": 1, "waves": 16, "tile_n": 32}, {"kernel": 1, "waves": 4, "split_k": 2}]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_fused_equals_two_step(gpu, m, dtype):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_matmul_quantize
    for n, k in ((256, 2048), (40, 1024), (1024, 8192)):
        raw, fields = weight(gpu, n, k, seed=n + k)
        gen = torch.Generator(device=gpu).manual_seed(1000 * m + k)
        x = (torch.randn((m, k), generator=gen, device=gpu) * 3).to(dtype)
        x[0, :32] = 0  # an all-zero group (exponent 0)
        for cfg in CONFIGS:
            step(f"fused M={m} {dtype} N={n} K={k} cfg={cfg}")
            fused = launch_iq3_s_matmul_quantize(x, fields, config=cfg)
            ref, (xv, xs) = two_step(x, fields, cfg)
            torch.cuda.synchronize()
            assert torch.equal(fused, ref), (n, k, cfg, float((fused - ref).abs().max()))
        expected = oracle.iq3s_fp8_matmul(xv.cpu().numpy(), xs.cpu().numpy(), raw)
        assert rel_l2(fused.cpu().numpy(), expected) <= 1e-3


def test_fused_grouped_strided_and_fallbacks(gpu):
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_matmul_quantize
    k = 4096
    parts = [weight(gpu, n, k, seed=7 + n) for n in (512, 128, 128)]
    fields = [f for _, f in parts]
    gen = torch.Generator(device=gpu).manual_seed(5)
    base = torch.randn((9, 2 * k + 8), generator=gen, device=gpu).to(torch.bfloat16)
    for m in (1, 3):
        x = base[:m, :k]  # row stride 2K+8 elements (16-byte aligned)
        step(f"fused grouped q/k/v-like M={m}, strided rows")
        outs = launch_iq3_s_matmul_quantize(x, fields)
        refs, _ = two_step(x.contiguous(), fields, None)
        torch.cuda.synchronize()
        assert all(torch.equal(o, r) for o, r in zip(outs, refs))
    x_odd = base[:2, 1:k + 1]  # base not 16-byte aligned: quantized in a launch of its own
    step("fused call, unaligned rows (two launches)")
    out = launch_iq3_s_matmul_quantize(x_odd, fields[0])
    ref, _ = two_step(x_odd.contiguous(), fields[0], None)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for m in (8, 33):  # dense / tiled families: quantizer, then the GEMM
        x = base[:m, :k] if m <= 9 else torch.randn((m, k), generator=gen, device=gpu).to(torch.bfloat16)
        step(f"fused call M={m} (two launches)")
        out = launch_iq3_s_matmul_quantize(x, fields[0])
        ref, (xv, xs) = two_step(x.contiguous(), fields[0], None)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert rel_l2(out.cpu().numpy(), oracle.iq3s_fp8_matmul(xv.cpu().numpy(), xs.cpu().numpy(), parts[0][0])) <= 1e-3


def test_fused_abi_leaves_mxfp8_buffers_alone_when_fused(gpu):
    """Through the C ABI: M <= 4 does not write xv/xs (one launch); M = 8 writes the
    quantizer's codes there."""
    from mambo_amd import _native
    from mambo_amd.kernels.iq3_s_fp8 import ensure_packed
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    k, n = 2048, 64
    _, fields = weight(gpu, n, k, seed=3)
    lib = _native.lib()
    for m, fused in ((2, True), (8, False)):
        x = torch.randn((m, k), device=gpu, dtype=torch.float32)
        xv = torch.full((m, k), 0xAB, dtype=torch.uint8, device=gpu)
        xs = torch.full((m, k // 32), 0xAB, dtype=torch.uint8, device=gpu)
        out = torch.empty((m, n), dtype=torch.float32, device=gpu)
        proj = (_native.Projection * 1)()
        proj[0] = _native.Projection(ensure_packed(fields, None).data_ptr(), n, out.data_ptr(), n)
        step(f"ABI fused call M={m}")
        rc = lib.mambo_iq3s_matmul_quantize_grouped(x.data_ptr(), _native.DTYPE_F32, k, m, proj, 1, k // 256, None,
                                                     xv.data_ptr(), k, xs.data_ptr(), k // 32,
                                                     _native.stream_handle(None))
        torch.cuda.synchronize()
        assert rc == 0, lib.mambo_last_error()
        qv, qs = launch_quantize_fp8(x)
        torch.cuda.synchronize()
        if fused:
            assert bool((xv == 0xAB).all()) and bool((xs == 0xAB).all())
        else:
            assert torch.equal(xv, qv) and torch.equal(xs, qs)
    bad = lib.mambo_iq3s_matmul_quantize_grouped(x.data_ptr(), 7, k, 1, proj, 1, k // 256, None, xv.data_ptr(), k,
                                                 xs.data_ptr(), k // 32, _native.stream_handle(None))
    assert bad == _native.MAMBO_ERR_VALUE
    with pytest.raises(ValueError, match="float32 or bfloat16"):
        from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_matmul_quantize
        launch_iq3_s_matmul_quantize(torch.zeros((1, k), dtype=torch.float16, device=gpu), fields)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_nonfinite_rows(gpu, dtype):
    """Rows holding NaN or +-inf, quantized inside the projection and by the quantizer
    launch: a row with a non-finite group (scale byte 0xFF, NaN codes) gives NaN in
    every output of that row on both paths; the finite rows are bit-identical."""
    from mambo_amd.kernels.iq3_s_fp8 import launch_iq3_s_matmul_quantize
    raw, fields = weight(gpu, 256, 2048, seed=77)
    gen = torch.Generator(device=gpu).manual_seed(77)
    x = torch.randn((4, 2048), generator=gen, device=gpu)
    x[1, 100] = float("inf")
    x[3, 2047] = float("nan")
    x[3, 5] = float("-inf")
    x = x.to(dtype)
    for cfg in CONFIGS:
        step(f"fused non-finite rows {dtype} cfg={cfg}")
        fused = launch_iq3_s_matmul_quantize(x, fields, config=cfg)
        ref, (xv, xs) = two_step(x, fields, cfg)
        torch.cuda.synchronize()
        assert torch.isnan(fused[[1, 3]]).all() and torch.isnan(ref[[1, 3]]).all(), cfg
        assert torch.equal(fused[[0, 2]], ref[[0, 2]]), cfg
        assert torch.isfinite(fused[[0, 2]]).all(), cfg
    assert int((xs.cpu() == 0xFF).sum()) == 3
