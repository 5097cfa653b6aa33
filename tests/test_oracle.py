"""Pins of the CPU oracle (no GPU): every check compares the oracle with something it
did not compute itself - a second published form of the codebook, brute force over
the E4M3 codes, float64 math, the reference tests' constructions and known answers."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import (GOLDEN, all_codes_blocks, e4m3_encode_bruteforce, e4m3_values,
                      make_synthetic_iq3_s)
from oracle import oracle


# ------------------------------------------------------------------------ codebook
def test_codebook_hex_table_matches_kgrid_512():
    """The product's iq3s_grid (hex words) against the oracle's table rebuilt from ggml's
    kgrid_512 (3-bit levels): two published forms of the same codebook."""
    from mambo_amd.kernels.iq3_s_fp8 import iq3_s_table
    product = iq3_s_table()
    from_kgrid = oracle.iq3s_grid()
    assert product.shape == from_kgrid.shape == (512,)
    np.testing.assert_array_equal(product, from_kgrid)
    assert np.all(np.diff(product.astype(np.int64)) > 0), "grid words are strictly ascending"
    mags = np.stack([(product >> s) & 0xFF for s in (0, 8, 16, 24)], axis=-1)
    assert set(np.unique(mags).tolist()) <= {1, 3, 5, 7, 9, 11, 13, 15}
    assert product[0] == 0x01010101 and product[-1] == 0x0F0F0101


def test_fp8_codebook_preserves_every_iq3_s_magnitude():
    """test_iq3_s_fp8.py:71-81: the E4M3-encoded codebook decodes to the magnitudes."""
    from mambo_amd.kernels.iq3_s_fp8 import iq3_s_fp8_table, iq3_s_table
    raw, enc = iq3_s_table(), iq3_s_fp8_table()
    assert raw.dtype == enc.dtype == np.uint32
    vals = e4m3_values()
    mags = np.stack([(raw >> s) & 0xFF for s in (0, 8, 16, 24)], axis=-1).astype(np.float64)
    bits = np.stack([(enc >> s) & 0xFF for s in (0, 8, 16, 24)], axis=-1).astype(np.uint8)
    np.testing.assert_array_equal(vals[bits], mags)
    np.testing.assert_array_equal(vals[bits | 0x80], -mags)


# ------------------------------------------------------------------------ E4M3
def test_e4m3_decode_all_codes():
    got = oracle.e4m3_decode_all().astype(np.float64)
    ref = e4m3_values()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == 2
    np.testing.assert_array_equal(got[~nan], ref[~nan])


def test_e4m3_encode_every_bf16_pattern():
    """All 65536 bf16 patterns (finite): nearest-even with saturation vs brute force.
    bf16 inputs put ties between E4M3 neighbours in every binade."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    x = (bits << 16).view(np.float32)
    x = x[np.isfinite(x)].astype(np.float64)
    np.testing.assert_array_equal(oracle.e4m3_encode(x), e4m3_encode_bruteforce(x))


def test_e4m3_encode_midpoints_and_random():
    vals = e4m3_values()[:127]
    mids = (vals[:-1] + vals[1:]) / 2
    eps = np.abs(mids) * 2.0 ** -40 + 2.0 ** -60
    rng = np.random.default_rng(7)
    rand = np.exp2(rng.uniform(-14, 10, 200_000)) * rng.choice([-1.0, 1.0], 200_000)
    x = np.concatenate([mids, mids - eps, mids + eps, -mids, vals, [448, 464, 464.0001, 1e30, -1e30, -0.0, 0.0],
                        rand])
    np.testing.assert_array_equal(oracle.e4m3_encode(x), e4m3_encode_bruteforce(x))


# ------------------------------------------------------------------------ MXFP8
def _exponent_f64(amax: np.ndarray) -> np.ndarray:
    """quantize_fp8.py:34-35 / fp8_reference.py:72-78 evaluated in float64."""
    a = amax.astype(np.float64)
    with np.errstate(divide="ignore"):
        e = np.ceil(np.log2(np.where(a > 0, a, 448.0) / 448.0))
    return np.clip(e, -127, 127).astype(np.int32)


def test_mxfp8_exponent_exact_over_all_binades():
    exps = np.arange(-149, 128)
    bases = []
    for e in exps:
        b = np.float32(2.0) ** np.float32(e) if e >= -126 else np.float32(2.0 ** float(e))
        bases.append(b)
    bases = np.array(bases, dtype=np.float32)
    mant = np.array([1.0, 1.5, 1.75, 1.9999999], dtype=np.float32)
    a = (bases[:, None] * mant[None, :]).ravel()
    with np.errstate(over="ignore"):
        a = np.concatenate([a, np.nextafter(a, np.float32(np.inf)), np.nextafter(a, np.float32(0))])
    rng = np.random.default_rng(3)
    a = np.concatenate([a, np.abs(rng.standard_normal(100_000).astype(np.float32)) * np.exp2(
        rng.integers(-140, 120, 100_000)).astype(np.float32), [0.0]]).astype(np.float32)
    a = a[np.isfinite(a)]
    np.testing.assert_array_equal(oracle.mxfp8_exponent(a), _exponent_f64(a))


def _numpy_quantizer(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """MXFP8 with float64 exponent and brute-force RNE codes, independent of the oracle."""
    m, k = x.shape
    g = x.reshape(m, k // 32, 32).astype(np.float64)
    amax = np.abs(x.reshape(m, k // 32, 32)).max(axis=2)
    e = _exponent_f64(amax)
    y = g / np.exp2(e.astype(np.float64))[..., None]
    q = e4m3_encode_bruteforce(y.ravel()).reshape(m, k)
    return q, (e + 127).astype(np.uint8)


def _reference_encode(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """encode_mxfp8_reference (fp8_reference.py:61-85): argmin over the finite codes,
    which breaks ties toward the smaller magnitude."""
    vals = e4m3_values()[:127]
    m, k = x.shape
    q = np.empty((m, k), dtype=np.uint8)
    s = np.empty((m, k // 32), dtype=np.uint8)
    for r in range(m):
        for b in range(k // 32):
            v = x[r, 32 * b:32 * b + 32]
            amax = float(np.max(np.abs(v)))
            e = 0 if amax == 0.0 else min(127, max(-127, int(np.ceil(np.log2(amax / 448.0)))))
            s[r, b] = e + 127
            nrm = v.astype(np.float64) / np.exp2(e)
            code = np.argmin(np.abs(np.abs(nrm)[:, None] - vals[None, :]), axis=1).astype(np.uint8)
            q[r, 32 * b:32 * b + 32] = code | np.where(np.signbit(nrm), 0x80, 0).astype(np.uint8)
    return q, s


def test_quantizer_reference_rows_known_answers():
    from golden.make_golden import quant_rows_input
    x = quant_rows_input()
    v, s = oracle.quantize_mxfp8(x)
    # zero row: e = 0, all codes +0
    assert np.all(s[0] == 127) and np.all(v[0] == 0)
    # 32.0 = 1.0 * 2^5 -> e = -3 (scale byte 124); 32 * 2^3 = 256 = 2^8 -> code 0x78
    assert s[1, 0] == 124 and v[1, 0] == 0x78
    # -64 = 1.0 * 2^6 -> e = -2 (125); -64 * 4 = -256 -> 0xF8
    assert s[2, 1] == 125 and v[2, 32 + 7] == 0xF8
    # 2^-130 (f32 subnormal): e clamps to -127 (scale byte 0); 2^-130 * 2^127 = 2^-3 -> 0x20
    assert s[3, 1] == 0 and np.all(v[3, 32:64] == 0x20)
    # linspace(-12, 12): amax 12 = 1.5 * 2^3 -> e = -5 (122); 12 * 32 = 384 -> 0x7C
    assert s[4, 2] == 122 and v[4, 64 + 31] == 0x7C and v[4, 64] == 0xFC
    qn, sn = _numpy_quantizer(x)
    np.testing.assert_array_equal(v, qn)
    np.testing.assert_array_equal(s, sn)


def test_quantizer_matches_reference_encoder_off_ties():
    rng = np.random.default_rng(20261015)
    x = rng.standard_normal((33, 160)).astype(np.float32)
    v, s = oracle.quantize_mxfp8(x)
    qr, sr = _reference_encode(x)
    np.testing.assert_array_equal(s, sr)
    vals = e4m3_values()[:127]
    mids = set(((vals[:-1] + vals[1:]) / 2).tolist())
    nrm = np.abs(x.astype(np.float64) / np.exp2(np.repeat(s.astype(np.int32) - 127, 32, axis=1)))
    tie = np.vectorize(lambda t: t in mids)(nrm)
    assert tie.sum() == 0  # random f32 data essentially never sits on a midpoint
    np.testing.assert_array_equal(v[~tie], qr[~tie])


def test_quantizer_ties_round_to_even():
    # In the binade [8, 16) E4M3 steps by 1. 8.5 ties 8 (even mantissa) and 9 -> 8;
    # 9.5 ties 9 (odd) and 10 (even) -> 10, where the reference's argmin encoder gives 9.
    x = np.zeros((1, 32), dtype=np.float32)
    x[0, :4] = [448.0, 8.5, 9.5, -9.5]
    v, s = oracle.quantize_mxfp8(x)
    assert s[0, 0] == 127
    vals = e4m3_values()
    assert vals[v[0, 1]] == 8.0 and vals[v[0, 2]] == 10.0 and vals[v[0, 3]] == -10.0


def nonfinite_rows() -> np.ndarray:
    """Rows with non-finite groups (the build's rule; outside the reference's tests):
    group 0 holds +inf among finite values, group 1 a NaN, group 2 -inf and a NaN,
    group 3 is finite (and must quantize as usual), group 4 only infinities."""
    x = np.random.default_rng(3).standard_normal((2, 160)).astype(np.float32)
    x[0, 5] = np.inf
    x[0, 32 + 9] = np.nan
    x[0, 64 + 1] = -np.inf
    x[0, 64 + 30] = np.nan
    x[0, 128:160] = np.where(np.arange(32) % 2, np.inf, -np.inf)
    x[1, 31] = -np.inf
    return x


def test_quantizer_nonfinite_groups_known_answers():
    """A group holding NaN or +-inf: scale byte 0xFF (E8M0 NaN) and, for each element,
    the E4M3 NaN 0x7F with the element's sign; every other group is unaffected."""
    x = nonfinite_rows()
    v, s = oracle.quantize_mxfp8(x)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    for r, g in ((0, 0), (0, 1), (0, 2), (0, 4), (1, 0)):
        assert s[r, g] == 0xFF, (r, g)
        np.testing.assert_array_equal(v[r, 32 * g:32 * g + 32], 0x7F | sign[r, 32 * g:32 * g + 32])
    finite = np.ones_like(s, dtype=bool)
    finite[0, [0, 1, 2, 4]] = False
    finite[1, 0] = False
    clean = np.where(np.isfinite(x), x, 0).astype(np.float32)
    cv, cs = oracle.quantize_mxfp8(clean)
    np.testing.assert_array_equal(s[finite], cs[finite])
    np.testing.assert_array_equal(v.reshape(2, 5, 32)[finite], cv.reshape(2, 5, 32)[finite])
    assert np.all(np.isnan(oracle.mxfp8_decode(v, s).reshape(2, 5, 32)[~finite]))


def test_bf16_input_equals_f32_input():
    bits = oracle.gen_bf16(5, 16 * 256, outlier_frac=0.01).reshape(16, 256)
    f = oracle.bf16_to_f32(bits)
    v1, s1 = oracle.quantize_mxfp8(bits)
    v2, s2 = oracle.quantize_mxfp8(f)
    np.testing.assert_array_equal(v1, v2)
    np.testing.assert_array_equal(s1, s2)


# ------------------------------------------------------------------------ IQ3_S decode
def test_decode_all_codes_and_sign_nibbles():
    """test_iq3_s_fp8.py:105-131: every index x every sign nibble, d = 1, scales 0;
    expected values come from the constructor's arrays and the grid, not from a decoder."""
    raw, code, sign = all_codes_blocks()
    grid = oracle.iq3s_grid()
    mags = np.stack([(grid[code] >> (8 * j)) & 0xFF for j in range(4)], axis=-1).astype(np.float32)
    sgn = np.stack([np.where((sign >> j) & 1, -1.0, 1.0) for j in range(4)], axis=-1).astype(np.float32)
    expected = (mags * sgn).reshape(8, -1)
    np.testing.assert_array_equal(oracle.dequant_iq3s(raw), expected)


def test_decode_scale_nibbles_and_d():
    """Known answers for the group scale: block with every code = index 0 (magnitudes 1),
    no signs, nibble s_g = g + 8 (g odd) or g, and d = 0.5 -> w = 0.5 * (1 + 2 s_g)."""
    raw = np.zeros((1, 1, 110), dtype=np.uint8)
    raw[0, 0, :2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    nib = np.array([0, 9, 2, 11, 4, 13, 6, 15], dtype=np.uint8)
    raw[0, 0, 106:110] = nib[0::2] | (nib[1::2] << 4)
    w = oracle.dequant_iq3s(raw).reshape(8, 32)
    np.testing.assert_array_equal(w, np.repeat((0.5 * (1 + 2 * nib.astype(np.float32)))[:, None], 32, axis=1))
    # one high bit: code 9 (group 1) takes index 256 and its first weight (36) is negative
    raw[0, 0, 66 + 1] = 0x02                 # qh bit of code 9 (bit 9 % 8 of qh[9 // 8])
    raw[0, 0, 74 + 36 // 8] = 1 << (36 % 8)  # sign of weight 36 = 4*9 + 0
    w = oracle.dequant_iq3s(raw)[0]
    g256 = int(oracle.iq3s_grid()[256])
    assert g256 == 0x05090507
    mags = np.array([(g256 >> (8 * j)) & 0xFF for j in range(4)], dtype=np.float32)
    f1 = 0.5 * (1 + 2 * 9)
    np.testing.assert_array_equal(w[36:40], mags * np.array([-1, 1, 1, 1], dtype=np.float32) * f1)
    np.testing.assert_array_equal(np.delete(w, np.arange(36, 40))[32:60], np.full(28, f1, np.float32))


def test_fp8_form_reconstructs_weights():
    raw = make_synthetic_iq3_s(5, 3 * 256, seed=0x1A3)
    bits, scales = oracle.dequant_iq3s_fp8(raw)
    vals = e4m3_values().astype(np.float32)
    np.testing.assert_array_equal(vals[bits] * np.repeat(scales, 32, axis=1), oracle.dequant_iq3s(raw))


def test_projection_matches_numpy_float64():
    raw = make_synthetic_iq3_s(7, 768, seed=0x3F8)
    x = np.random.default_rng(20261016).standard_normal((9, 768)).astype(np.float32)
    xv, xs = oracle.quantize_mxfp8(x)
    out = oracle.iq3s_fp8_matmul(xv, xs, raw)
    xe = oracle.mxfp8_decode(xv, xs).astype(np.float64)
    w = oracle.dequant_iq3s(raw).astype(np.float64)
    np.testing.assert_allclose(out, (xe @ w.T).astype(np.float32), rtol=1e-6, atol=1e-7)
    # decoded activations equal e4m3 value * 2^(s-127) exactly
    np.testing.assert_array_equal(xe, e4m3_values()[xv] * np.exp2(np.repeat(xs.astype(np.float64) - 127, 32, 1)))


# ------------------------------------------------------------------------ generators
def test_generators_are_counter_based():
    a = oracle.gen_iq3s(0, 6, 4)
    b = oracle.gen_iq3s(0, 2, 4, row0=3)
    np.testing.assert_array_equal(a[3:5], b)
    d = a[..., :2].copy().view(np.float16).astype(np.float32)
    assert np.all(np.isfinite(d)) and np.all(d >= 0) and d.max() < 0.013
    x = oracle.gen_bf16(1, 1000)
    np.testing.assert_array_equal(oracle.gen_bf16(1, 10, start=500), x[500:510])
    f = oracle.bf16_to_f32(oracle.gen_bf16(1, 200_000))
    assert abs(float(f.mean())) < 0.01 and abs(float(f.std()) - 1.0) < 0.01
    fo = oracle.bf16_to_f32(oracle.gen_bf16(1, 200_000, outlier_frac=0.001))
    n_out = int(np.sum(np.abs(fo) > 10))
    assert 100 < n_out < 320


# ------------------------------------------------------------------------ fixtures
@pytest.mark.parametrize("name", ["quant_rows", "quant_bf16_outliers", "decode_random", "matmul_small"])
def test_oracle_reproduces_golden_fixture(name):
    g = np.load(GOLDEN / f"{name}.npz")
    if name == "quant_rows":
        v, s = oracle.quantize_mxfp8(g["x"])
        np.testing.assert_array_equal(v, g["values"])
        np.testing.assert_array_equal(s, g["scales"])
    elif name == "quant_bf16_outliers":
        v, s = oracle.quantize_mxfp8(g["x_bf16"])
        np.testing.assert_array_equal(v, g["values"])
        np.testing.assert_array_equal(s, g["scales"])
    elif name == "decode_random":
        bits, sc = oracle.dequant_iq3s_fp8(g["raw"])
        np.testing.assert_array_equal(bits, g["values"])
        np.testing.assert_array_equal(sc, g["scales"])
        np.testing.assert_array_equal(oracle.dequant_iq3s(g["raw"]), g["weights"])
    else:
        np.testing.assert_array_equal(oracle.iq3s_fp8_matmul(g["x_values"], g["x_scales"], g["raw"]), g["out"])
