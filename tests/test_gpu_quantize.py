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


def test_hardware_e4m3_path(gpu):
    """The quantizer's rounding (kQuantHwCvt: the hardware v_cvt_pk_fp8_f32) on every
    value it can be fed, |y| <= 448: (1) all 2 x 1.14e9 float32 bit patterns in that
    range through the hardware and the integer software path, compared on the GPU;
    (2) every bf16 pattern in the range, every E4M3 midpoint (the ties) and the floats
    next to them, hardware path against the oracle."""
    from conftest import e4m3_values
    from mambo_amd import _native
    lib = _native.lib()
    top = 0x43E00000  # 448.0f
    chunk = 1 << 27
    sw = torch.empty(chunk, dtype=torch.uint8, device=gpu)
    hw = torch.empty(chunk, dtype=torch.uint8, device=gpu)
    for sign in (0, -(1 << 31)):
        step(f"e4m3 hardware vs software, every f32 pattern |x| <= 448, sign bit {int(sign != 0)}")
        for lo in range(0, top + 1, chunk):
            hi = min(lo + chunk, top + 1)
            bits = torch.arange(lo, hi, dtype=torch.int32, device=gpu) | sign
            n = hi - lo
            _native.check(lib.mambo_e4m3_convert(bits.data_ptr(), n, sw.data_ptr(), hw.data_ptr(),
                                                 _native.stream_handle(None)))
            if not torch.equal(sw[:n], hw[:n]):
                bad = torch.nonzero(sw[:n] != hw[:n])[:5, 0]
                raise AssertionError(f"hardware and software E4M3 differ at f32 bits "
                                     f"{[hex((int(b) + lo) | (sign & 0xFFFFFFFF)) for b in bad]}")
        torch.cuda.synchronize()
    bf16 = np.arange(0, 0x43E1, dtype=np.uint32) << 16
    vals = e4m3_values()[:127]
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    x = np.concatenate([bf16.view(np.float32), mids, np.nextafter(mids, np.float32(0)),
                        np.nextafter(mids, np.float32(1e9)), vals.astype(np.float32)])
    x = np.concatenate([x, -x]).astype(np.float32)
    xt = torch.from_numpy(x).to(gpu)
    out = torch.empty(x.size, dtype=torch.uint8, device=gpu)
    step(f"e4m3 hardware path against the oracle on {x.size} values")
    _native.check(lib.mambo_e4m3_convert(xt.data_ptr(), x.size, None, out.data_ptr(), _native.stream_handle(None)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.e4m3_encode(x.astype(np.float64)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_nonfinite_groups(gpu, dtype):
    """Groups holding NaN or +-inf: scale byte 0xFF and E4M3 NaN codes with the input's
    signs; the other groups of the same rows quantize as usual (oracle rule)."""
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    from test_oracle import nonfinite_rows
    x = torch.from_numpy(nonfinite_rows()).to(gpu).to(dtype)
    step(f"quantize non-finite rows {dtype}")
    q, s = launch_quantize_fp8(x)
    torch.cuda.synchronize()
    host = x.cpu()
    eq, es = oracle.quantize_mxfp8(host.numpy() if dtype == torch.float32 else host.view(torch.int16).numpy()
                                   .view(np.uint16))
    np.testing.assert_array_equal(s.cpu().numpy(), es)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    assert (es == 0xFF).sum() == 5
