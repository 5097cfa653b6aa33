"""MXFP8 quantizer on the GPU against the CPU oracle: bit-exact codes and scales."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import oracle

pytestmark = pytest.mark.gpu


def step(msg: str) -> None:
    print(f"[gpu] {msg}", flush=True)


@pytest.mark.parametrize("tokens", [5, 33, 128])
def test_f32_to_mxfp8_quantization_matches_oracle(gpu, tokens):
    """test_iq3_s_fp8.py:151-175 rows (zero row, 32.0, -64.0, x1e-4, 2^-130, linspace)."""
    from golden.make_golden import quant_rows_input
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    x = quant_rows_input(tokens)
    step(f"quantize f32 [{tokens},160]")
    q, s = launch_quantize_fp8(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert q.dtype == np.uint8 and q.shape == (tokens, 160)
    assert s.dtype == np.uint8 and s.shape == (tokens, 5)
    eq, es = oracle.quantize_mxfp8(x)
    np.testing.assert_array_equal(q, eq)
    np.testing.assert_array_equal(s, es)
    assert np.all(q[0] == 0) and np.all(s[0] == 127)
    if tokens == 5:
        g = np.load(GOLDEN / "quant_rows.npz")
        np.testing.assert_array_equal(q, g["values"])
        np.testing.assert_array_equal(s, g["scales"])


def test_bf16_golden_fixture(gpu):
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    g = np.load(GOLDEN / "quant_bf16_outliers.npz")
    x = torch.from_numpy(g["x_bf16"].astype(np.int16)).view(torch.bfloat16).to(gpu)
    step("quantize bf16 golden [8,512]")
    q, s = launch_quantize_fp8(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), g["values"])
    np.testing.assert_array_equal(s.cpu().numpy(), g["scales"])


def test_quantizer_config_bf16_4096_with_outliers(gpu):
    """bf16 [4096, 4096] ~N(0,1) with 0.1% x100 outliers (seeded positions): bit-exact.
    Inputs come from the GPU generator; a sample is checked against the oracle's."""
    from mambo_amd import _native
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    m = k = 4096
    bits = torch.empty(m * k, dtype=torch.int16, device=gpu)
    step("synth bf16 [4096,4096]")
    _native.check(_native.lib().mambo_synth_bf16(1, 2, 0.001, 0, m * k, bits.data_ptr(),
                                                 _native.stream_handle(None)))
    x = bits.view(torch.bfloat16).view(m, k)
    step("quantize bf16 [4096,4096]")
    q, s = launch_quantize_fp8(x)
    torch.cuda.synchronize()
    xb = bits.cpu().numpy().view(np.uint16).reshape(m, k)
    np.testing.assert_array_equal(xb.ravel()[:65536], oracle.gen_bf16(1, 65536, outlier_seed=2, outlier_frac=0.001))
    n_out = int(np.sum(np.abs(oracle.bf16_to_f32(xb)) > 12.0))
    assert 0.0005 * m * k < n_out < 0.002 * m * k
    eq, es = oracle.quantize_mxfp8(xb)
    np.testing.assert_array_equal(s.cpu().numpy(), es)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)


def test_strided_rows_and_dtype_equivalence(gpu):
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((17, 1024)) * np.exp2(rng.integers(-20, 20, (17, 1)))).astype(np.float32)
    xg = torch.from_numpy(x).to(gpu)
    big = torch.zeros((17, 1536), dtype=torch.float32, device=gpu)
    big[:, 256:1280] = xg
    step("quantize strided f32 / bf16 [17,1024]")
    q1, s1 = launch_quantize_fp8(xg)
    q2, s2 = launch_quantize_fp8(big[:, 256:1280])          # row stride 1536
    q3, s3 = launch_quantize_fp8(xg.to(torch.bfloat16))
    q4, s4 = launch_quantize_fp8(xg.to(torch.bfloat16).float())
    xt = torch.zeros((1024, 17), dtype=torch.float32, device=gpu)
    xt.copy_(xg.t())
    q5, s5 = launch_quantize_fp8(xt.t())                    # column stride 17: copied first
    torch.cuda.synchronize()
    eq, es = oracle.quantize_mxfp8(x)
    for q, s in ((q1, s1), (q2, s2), (q5, s5)):
        np.testing.assert_array_equal(q.cpu().numpy(), eq)
        np.testing.assert_array_equal(s.cpu().numpy(), es)
    np.testing.assert_array_equal(q3.cpu().numpy(), q4.cpu().numpy())
    np.testing.assert_array_equal(s3.cpu().numpy(), s4.cpu().numpy())


def test_software_e4m3_path_matches_oracle(gpu):
    """The kernels' integer E4M3 rounding against the oracle on ties, midpoints,
    subnormals and random values (the quantizer feeds it |y| <= 448)."""
    from mambo_amd import _native
    from conftest import e4m3_values
    vals = e4m3_values()[:127]
    mids = (vals[:-1] + vals[1:]) / 2
    rng = np.random.default_rng(5)
    rand = np.exp2(rng.uniform(-16, 9, 1 << 20)) * rng.choice([-1.0, 1.0], 1 << 20)
    x = np.concatenate([vals, -vals, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9), rand,
                        [0.0, -0.0, 448.0, 2.0 ** -10, 3 * 2.0 ** -11]]).astype(np.float32)
    xt = torch.from_numpy(x).to(gpu)
    sw = torch.empty(x.size, dtype=torch.uint8, device=gpu)
    step(f"e4m3 software conversion of {x.size} values")
    _native.check(_native.lib().mambo_e4m3_convert(xt.data_ptr(), x.size, sw.data_ptr(), None,
                                                   _native.stream_handle(None)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sw.cpu().numpy(), oracle.e4m3_encode(x.astype(np.float64)))
