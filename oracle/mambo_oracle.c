/*
 * CPU oracle for the fused IQ3_S x MXFP8 projection path.
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, in plain C, the arithmetic of
 * the reference path so that the HIP product can be checked against it. Only
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load
 * the library built from it, and only to check results or as the timed CPU
 * baseline; the product (mambo_amd/) never links, imports or calls it.
 *
 * What each part follows (paths are in the Menooker/Mambo reference):
 *   - IQ3_S block layout and decode: src/python/mambo/kernels/iq3_s_fp8.py:11-21,
 *     105-199 and llama.cpp's dequantize_row_iq3_s (called by
 *     tests/cpp/reference/ggml_reference.cpp:508 through traits->to_float).
 *   - FP8-form decode (E4M3 bits + f32 group scales): iq3_s_fp8.py:77-94,186-222,341-351.
 *   - MXFP8 activation quantizer: src/python/mambo/kernels/quantize_fp8.py:23-39
 *     (kernel semantics: round-to-nearest-even, saturating) and the codecs of
 *     tests/python/utils/fp8_reference.py:10-85.
 *   - CPU projection: ggml_reference.cpp:495-523 (to_float of each weight row,
 *     then a float64-accumulated dot product, cast to f32) and
 *     tests/python/utils/compute_reference_gguf.py:111-121.
 *   - Codebook: llama.cpp (Menooker/llama.cpp-adaptive-kv-streaming @ 21b359d8)
 *     ggml-quants.c kgrid_512 -> iq3s_grid via iq3xs_init_impl(512); the
 *     submodule is absent, see iq3s_kgrid_512 below.
 *
 * Parity pins (all exercised by tests/test_oracle.py):
 *   - codebook: kgrid_512 (here) == the product's hex iq3s_grid table, entry by entry;
 *   - E4M3 codec: exhaustive encode/decode against brute-force nearest-even over
 *     the 126 finite positive codes (numpy, independent of this file);
 *   - MXFP8 exponent: exact rule vs float64 ceil(log2(amax/448)) over all f32 exponents;
 *   - quantizer: the reference's special rows (test_iq3_s_fp8.py:155-161) as
 *     known answers, and a numpy port of encode_mxfp8_reference on non-tie elements;
 *   - IQ3_S decode: all 512 codes x 16 sign nibbles (test_iq3_s_fp8.py:105-131
 *     constructor), scale nibbles, and d, against expectations built from the
 *     block layout by a separate numpy decoder;
 *   - projection: f64 dot vs numpy f64 matmul of the decoded operands.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define IQ3S_BLOCK_BYTES 110
#define IQ3S_BLOCK_VALUES 256

/* ggml-quants.c kgrid_512 (iq3xs_init_impl, grid_size 512): each entry packs four
 * 3-bit levels l_j (bits 3j..3j+2); the grid magnitude of weight j is 2*l_j+1. */
static const uint16_t iq3s_kgrid_512[512] = {
    0, 1, 2, 5, 7, 8, 9, 10, 12, 14, 16, 17, 21, 27, 32, 34,
    37, 39, 41, 43, 48, 50, 57, 60, 63, 64, 65, 66, 68, 72, 73, 77,
    80, 83, 87, 89, 93, 100, 113, 117, 122, 128, 129, 133, 135, 136, 139, 142,
    145, 149, 152, 156, 162, 165, 167, 169, 171, 184, 187, 195, 201, 205, 208, 210,
    217, 219, 222, 228, 232, 234, 247, 249, 253, 256, 267, 271, 273, 276, 282, 288,
    291, 297, 312, 322, 324, 336, 338, 342, 347, 353, 357, 359, 374, 379, 390, 393,
    395, 409, 426, 441, 448, 450, 452, 464, 466, 470, 475, 488, 492, 512, 513, 514,
    516, 520, 521, 523, 525, 527, 528, 530, 537, 540, 542, 556, 558, 561, 570, 576,
    577, 579, 582, 584, 588, 593, 600, 603, 609, 616, 618, 632, 638, 640, 650, 653,
    655, 656, 660, 666, 672, 675, 685, 688, 698, 705, 708, 711, 712, 715, 721, 727,
    728, 732, 737, 754, 760, 771, 773, 778, 780, 793, 795, 802, 806, 808, 812, 833,
    840, 843, 849, 856, 858, 873, 912, 916, 919, 932, 934, 961, 963, 968, 970, 977,
    989, 993, 1010, 1016, 1024, 1025, 1027, 1029, 1031, 1032, 1034, 1036, 1038, 1041, 1043, 1047,
    1048, 1050, 1057, 1059, 1061, 1064, 1066, 1079, 1080, 1083, 1085, 1088, 1090, 1096, 1099, 1103,
    1106, 1109, 1113, 1116, 1122, 1129, 1153, 1156, 1159, 1169, 1171, 1176, 1183, 1185, 1195, 1199,
    1209, 1212, 1216, 1218, 1221, 1225, 1234, 1236, 1241, 1243, 1250, 1256, 1270, 1281, 1287, 1296,
    1299, 1306, 1309, 1313, 1338, 1341, 1348, 1353, 1362, 1375, 1376, 1387, 1400, 1408, 1410, 1415,
    1425, 1453, 1457, 1477, 1481, 1494, 1496, 1507, 1512, 1538, 1545, 1547, 1549, 1551, 1554, 1561,
    1563, 1565, 1570, 1572, 1575, 1577, 1587, 1593, 1601, 1603, 1605, 1612, 1617, 1619, 1632, 1648,
    1658, 1662, 1664, 1674, 1680, 1690, 1692, 1704, 1729, 1736, 1740, 1745, 1747, 1751, 1752, 1761,
    1763, 1767, 1773, 1787, 1795, 1801, 1806, 1810, 1817, 1834, 1840, 1844, 1857, 1864, 1866, 1877,
    1882, 1892, 1902, 1915, 1934, 1953, 1985, 1987, 2000, 2002, 2013, 2048, 2052, 2058, 2064, 2068,
    2071, 2074, 2081, 2088, 2104, 2114, 2119, 2121, 2123, 2130, 2136, 2141, 2147, 2153, 2157, 2177,
    2179, 2184, 2189, 2193, 2203, 2208, 2223, 2226, 2232, 2244, 2249, 2251, 2256, 2258, 2265, 2269,
    2304, 2306, 2324, 2335, 2336, 2361, 2373, 2375, 2385, 2418, 2443, 2460, 2480, 2504, 2509, 2520,
    2531, 2537, 2562, 2568, 2572, 2578, 2592, 2596, 2599, 2602, 2614, 2620, 2625, 2627, 2629, 2634,
    2641, 2650, 2682, 2688, 2697, 2707, 2712, 2718, 2731, 2754, 2759, 2760, 2775, 2788, 2793, 2805,
    2811, 2817, 2820, 2832, 2842, 2854, 2890, 2902, 2921, 2923, 2978, 3010, 3012, 3026, 3081, 3083,
    3085, 3097, 3099, 3120, 3136, 3152, 3159, 3188, 3210, 3228, 3234, 3245, 3250, 3256, 3264, 3276,
    3281, 3296, 3349, 3363, 3378, 3392, 3395, 3420, 3440, 3461, 3488, 3529, 3531, 3584, 3588, 3591,
    3600, 3602, 3614, 3616, 3628, 3634, 3650, 3657, 3668, 3683, 3685, 3713, 3716, 3720, 3726, 3729,
    3736, 3753, 3778, 3802, 3805, 3819, 3841, 3845, 3851, 3856, 3880, 3922, 3938, 3970, 3993, 4032,
};

static uint32_t g_grid[512];
static int g_grid_ready = 0;

/* iq3xs_init_impl(512): grid byte j of entry i is 2*((kgrid[i] >> 3j) & 7) + 1. */
void orc_iq3s_grid(uint32_t *out)
{
    for (int i = 0; i < 512; ++i) {
        uint32_t w = 0;
        for (int j = 0; j < 4; ++j) {
            uint32_t l = (iq3s_kgrid_512[i] >> (3 * j)) & 7u;
            w |= (2u * l + 1u) << (8 * j);
        }
        out[i] = w;
    }
}

static const uint32_t *grid(void)
{
    if (!g_grid_ready) {
        orc_iq3s_grid(g_grid);
        g_grid_ready = 1;
    }
    return g_grid;
}

/* ---------------------------------------------------------------- fp16 / bf16 */

float orc_fp16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15);
    int exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    double v;
    if (exp == 0)
        v = ldexp((double)man, -24);
    else if (exp == 31)
        v = man ? NAN : INFINITY;
    else
        v = ldexp((double)(man | 0x400u), exp - 25);
    return (float)(sign ? -v : v);
}

/* IEEE binary32 -> binary16, round to nearest even, overflow to infinity. */
uint16_t orc_f32_to_fp16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    int e = (int)(ax >> 23) - 127;
    uint32_t m = (ax & 0x7fffffu) | (ax >= 0x800000u ? 0x800000u : 0u);
    if (ax < 0x800000u)
        e = -126;
    if (e > 15)
        return (uint16_t)(sign | 0x7c00u);
    int shift; /* number of low bits of m to drop */
    uint32_t base;
    if (e >= -14) {
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
        m &= 0x7fffffu; /* implicit bit carried by the exponent field */
    } else {
        shift = 13 + (-14 - e);
        base = 0;
        if (shift > 24)
            return (uint16_t)sign;
    }
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u)))
        q += 1u;
    return (uint16_t)(sign | (base + q)); /* carries roll into the exponent */
}

uint16_t orc_f32_to_bf16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t h)
{
    uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------- E4M3 / E8M0
 * OCP FP8 E4M3 ("fn"): bias 7, no infinities, S.1111.111 is NaN, max 448.
 * fp8_reference.py:30-43 (decode). */
float orc_e4m3_decode(uint8_t b)
{
    int e = (b >> 3) & 0xf;
    int m = b & 7;
    double v;
    if (e == 0)
        v = m * ldexp(1.0, -9);
    else if (e == 15 && m == 7)
        v = NAN;
    else
        v = (1.0 + m / 8.0) * ldexp(1.0, e - 7);
    return (float)((b & 0x80) ? -v : v);
}

/* Round |y| to the E4M3 grid, nearest with ties to even, saturating at 448;
 * the sign of y (including -0) goes to bit 7. NaN input is out of contract. */
uint8_t orc_e4m3_encode(double y)
{
    uint8_t sign = signbit(y) ? 0x80 : 0x00;
    double a = fabs(y);
    if (a >= 464.0) /* halfway between 448 and the next binade step: saturate */
        return (uint8_t)(sign | 0x7e);
    if (a < ldexp(1.0, -6)) {
        /* subnormal grid step 2^-9; q == 8 is exactly the smallest normal (code 0x08) */
        double q = nearbyint(a * 512.0);
        return (uint8_t)(sign | (uint8_t)q);
    }
    int e2;
    double f = frexp(a, &e2); /* a = f * 2^e2, f in [0.5, 1) */
    int e = e2 - 1;            /* a = m * 2^e, m in [1, 2) */
    double mant = nearbyint((2.0 * f - 1.0) * 8.0);
    if (mant >= 8.0) {
        mant = 0.0;
        e += 1;
    }
    int code = ((e + 7) << 3) | (int)mant;
    if (code > 0x7e)
        code = 0x7e;
    return (uint8_t)(sign | code);
}

/* MXFP8 block exponent, quantize_fp8.py:32-38: e = max(ceil(log2(amax/448)), -127),
 * e = 0 for an all-zero block. Computed exactly from the bits: with
 * amax = m * 2^E (m in [1,2)), e = E-8 if m <= 1.75 else E-7. */
int orc_mxfp8_exponent(float amax)
{
    if (amax == 0.0f)
        return 0;
    int e2;
    double f = frexp((double)amax, &e2); /* amax = f * 2^e2, f in [0.5,1) */
    int e = (f <= 0.875) ? e2 - 9 : e2 - 8;
    if (e < -127)
        e = -127;
    if (e > 127)
        e = 127;
    return e;
}

/* Non-finite input is outside the reference's tests (fp8_reference.py:73-77 raises on
 * it, ggml_reference.cpp:458-460 rejects it). The build's rule: a group holding a NaN
 * or an infinity gets the E8M0 NaN scale 0xFF and, for every element, the E4M3 NaN
 * 0x7F with the element's sign. */
static void quantize_group(const float *v, uint8_t *q, uint8_t *s)
{
    int finite = 1;
    for (int i = 0; i < 32; ++i)
        finite &= isfinite(v[i]) != 0;
    if (!finite) {
        *s = 0xFF;
        for (int i = 0; i < 32; ++i)
            q[i] = (uint8_t)(0x7F | (signbit(v[i]) ? 0x80 : 0x00));
        return;
    }
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float a = fabsf(v[i]);
        if (a > amax)
            amax = a;
    }
    int e = orc_mxfp8_exponent(amax);
    *s = (uint8_t)(e + 127);
    double inv = ldexp(1.0, -e); /* exact power of two */
    for (int i = 0; i < 32; ++i)
        q[i] = orc_e4m3_encode((double)v[i] * inv);
}

/* x f32 [m, ldx] -> values u8 [m, k] (E4M3), scales u8 [m, k/32] (E8M0). */
void orc_quantize_mxfp8_f32(const float *x, int64_t m, int64_t k, int64_t ldx,
                            uint8_t *values, uint8_t *scales)
{
    for (int64_t r = 0; r < m; ++r)
        for (int64_t g = 0; g < k / 32; ++g)
            quantize_group(x + r * ldx + 32 * g, values + r * k + 32 * g, scales + r * (k / 32) + g);
}

void orc_quantize_mxfp8_bf16(const uint16_t *x, int64_t m, int64_t k, int64_t ldx,
                             uint8_t *values, uint8_t *scales)
{
    float tmp[32];
    for (int64_t r = 0; r < m; ++r)
        for (int64_t g = 0; g < k / 32; ++g) {
            for (int i = 0; i < 32; ++i)
                tmp[i] = orc_bf16_to_f32(x[r * ldx + 32 * g + i]);
            quantize_group(tmp, values + r * k + 32 * g, scales + r * (k / 32) + g);
        }
}

/* MXFP8 -> f32: e4m3(q) * 2^(s-127); exact in f32 except below 2^-149. Scale byte
 * 0xFF is the E8M0 NaN. */
void orc_mxfp8_decode(const uint8_t *values, const uint8_t *scales, int64_t m, int64_t k, float *out)
{
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < k; ++c) {
            const int s = scales[r * (k / 32) + c / 32];
            out[r * k + c] = s == 0xFF ? NAN : (float)ldexp((double)orc_e4m3_decode(values[r * k + c]), s - 127);
        }
}

/* ------------------------------------------------------------------- IQ3_S */

/* One 110-byte block -> 256 floats: llama.cpp dequantize_row_iq3_s.
 * w[4c+j] = f32(d) * (1 + 2*s_{c/8}) * byte_j(grid[qs[c] | qh_bit(c) << 8]) * sign,
 * qh bit of code c: bit c%8 of qh[c/8]; sign of weight w: bit w%8 of signs[w/8];
 * s_g: low nibble of scales[g/2] for even g, high nibble for odd g. */
static void dequant_block(const uint8_t *blk, float *y)
{
    const uint32_t *g = grid();
    uint16_t dh = (uint16_t)(blk[0] | (blk[1] << 8));
    float d = orc_fp16_to_f32(dh);
    const uint8_t *qs = blk + 2, *qh = blk + 66, *signs = blk + 74, *sc = blk + 106;
    for (int grp = 0; grp < 8; ++grp) {
        int s = (grp & 1) ? (sc[grp / 2] >> 4) : (sc[grp / 2] & 0xf);
        float db = d * (float)(1 + 2 * s);
        for (int c8 = 0; c8 < 8; ++c8) {
            int c = grp * 8 + c8;
            uint32_t idx = qs[c] | (((qh[c / 8] >> (c % 8)) & 1u) << 8);
            uint32_t gw = g[idx];
            for (int j = 0; j < 4; ++j) {
                int w = 4 * c + j;
                float mag = (float)((gw >> (8 * j)) & 0xffu);
                float v = db * mag;
                y[w] = ((signs[w / 8] >> (w % 8)) & 1) ? -v : v;
            }
        }
    }
}

/* raw u8 [n, nb, 110] (contiguous) -> out f32 [n, nb*256]. */
void orc_dequant_iq3s(const uint8_t *raw, int64_t n, int64_t nb, float *out)
{
    for (int64_t r = 0; r < n; ++r)
        for (int64_t b = 0; b < nb; ++b)
            dequant_block(raw + (r * nb + b) * IQ3S_BLOCK_BYTES, out + (r * nb + b) * IQ3S_BLOCK_VALUES);
}

/* E4M3 encodings of the odd grid magnitudes 1..15 (iq3_s_fp8.py:80-81). */
static uint8_t e4m3_of_small_odd(uint32_t mag)
{
    return orc_e4m3_encode((double)mag);
}

/* FP8 form of launch_dequant_iq3_s: values u8 [n, nb*256] = E4M3 of sign*grid byte,
 * scales f32 [n, nb*8] = f32(d) * (1 + 2*s). */
void orc_dequant_iq3s_fp8(const uint8_t *raw, int64_t n, int64_t nb, uint8_t *values, float *scales)
{
    const uint32_t *g = grid();
    for (int64_t r = 0; r < n; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *blk = raw + (r * nb + b) * IQ3S_BLOCK_BYTES;
            uint16_t dh = (uint16_t)(blk[0] | (blk[1] << 8));
            float d = orc_fp16_to_f32(dh);
            const uint8_t *qs = blk + 2, *qh = blk + 66, *signs = blk + 74, *sc = blk + 106;
            uint8_t *vo = values + (r * nb + b) * 256;
            float *so = scales + (r * nb + b) * 8;
            for (int grp = 0; grp < 8; ++grp) {
                int s = (grp & 1) ? (sc[grp / 2] >> 4) : (sc[grp / 2] & 0xf);
                so[grp] = d * (float)(1 + 2 * s);
            }
            for (int c = 0; c < 64; ++c) {
                uint32_t idx = qs[c] | (((qh[c / 8] >> (c % 8)) & 1u) << 8);
                for (int j = 0; j < 4; ++j) {
                    int w = 4 * c + j;
                    uint8_t code = e4m3_of_small_odd((g[idx] >> (8 * j)) & 0xffu);
                    vo[w] = (uint8_t)(code | ((((signs[w / 8] >> (w % 8)) & 1) != 0) ? 0x80 : 0));
                }
            }
        }
}

/* ---------------------------------------------------------------- projections */

/* out[m, n] = f32(sum_k f64(x[m,k]) * f64(w[n,k])), compute_reference_gguf.py:111-121. */
void orc_matmul_f64(const float *x, int64_t m, int64_t k, const float *w, int64_t n, float *out)
{
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (int64_t t = 0; t < k; ++t)
                acc += (double)x[i * k + t] * (double)w[j * k + t];
            out[i * n + j] = (float)acc;
        }
}

/* The reference CPU path of ggml_reference.cpp:495-523 applied to MXFP8 activations:
 * for each weight row: to_float (dequantize_row_iq3_s), then a double-accumulated dot
 * with every activation row (activations decoded from E4M3 + E8M0), cast to f32.
 * xv u8 [m, ldxv], xs u8 [m, ldxs]; raw u8 [n, nb, 110] contiguous; out f32 [m, n].
 * rows [row_begin, row_end) of the weight only (so a bounded sample can be timed). */
void orc_iq3s_fp8_matmul(const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t m,
                         const uint8_t *raw, int64_t n, int64_t nb, int64_t row_begin, int64_t row_end,
                         float *out, int threads)
{
    int64_t k = nb * 256;
    float *xf = (float *)malloc(sizeof(float) * (size_t)(m * k));
    for (int64_t i = 0; i < m; ++i)
        for (int64_t t = 0; t < k; ++t)
            xf[i * k + t] = (float)ldexp((double)orc_e4m3_decode(xv[i * ldxv + t]),
                                         (int)xs[i * ldxs + t / 32] - 127);
    (void)grid();
#ifdef _OPENMP
    if (threads > 0)
        omp_set_num_threads(threads);
#pragma omp parallel
#endif
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)k);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t r = row_begin; r < row_end; ++r) {
            for (int64_t b = 0; b < nb; ++b)
                dequant_block(raw + (r * nb + b) * IQ3S_BLOCK_BYTES, row + b * 256);
            for (int64_t i = 0; i < m; ++i) {
                double acc = 0.0;
                const float *xr = xf + i * k;
                for (int64_t t = 0; t < k; ++t)
                    acc += (double)row[t] * (double)xr[t];
                out[i * n + r] = (float)acc;
            }
        }
        free(row);
    }
    (void)threads;
    free(xf);
}

/* ----------------------------------------------------------------- generators
 * Counter-based synthetic inputs: any element can be regenerated independently,
 * so sampled rows of a multi-GB weight can be rebuilt on the CPU bit for bit.
 *   splitmix64 (Steele, Lea, Flood 2014 / Vigna):
 *     z += 0x9E3779B97F4A7C15; z = (z^(z>>30))*0xBF58476D1CE4E5B9;
 *     z = (z^(z>>27))*0x94D049BB133111EB; return z^(z>>31)
 *   rnd(seed, stream, ctr) = splitmix64(splitmix64(seed*0xD1B54A32D192ED03 + stream) + ctr)
 *   normal(seed, stream, i): Irwin-Hall sum of 12 uniforms, exact in double:
 *     (sum_{t<12} (rnd(seed, stream, 12i+t) >> 32) - 6*2^32) / 2^32
 */
static uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_rnd(uint64_t seed, uint64_t stream, uint64_t ctr)
{
    return splitmix64(splitmix64(seed * 0xD1B54A32D192ED03ull + stream) + ctr);
}

double orc_normal(uint64_t seed, uint64_t stream, uint64_t i)
{
    uint64_t key = splitmix64(seed * 0xD1B54A32D192ED03ull + stream);
    uint64_t s = 0;
    for (int t = 0; t < 12; ++t)
        s += splitmix64(key + 12 * i + (uint64_t)t) >> 32;
    return (double)((int64_t)s - (int64_t)(6ull << 32)) / 4294967296.0;
}

/* Random IQ3_S blocks for rows [row0, row0+nrows) of an [n_total, nb] weight:
 * bytes 2..109 of block (r, b) are bytes of rnd(seed, 1, 14*(r*nb+b) + j/8) (byte j%8),
 * d = fp16(f32(|normal(seed, 2, r*nb+b)| * 2e-3)). Output u8 [nrows, nb, 110]. */
void orc_gen_iq3s(uint64_t seed, int64_t nb, int64_t row0, int64_t nrows, uint8_t *raw)
{
    uint64_t key = splitmix64(seed * 0xD1B54A32D192ED03ull + 1);
    for (int64_t r = 0; r < nrows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            uint64_t blk = (uint64_t)((row0 + r) * nb + b);
            uint8_t *o = raw + (r * nb + b) * IQ3S_BLOCK_BYTES;
            for (int w = 0; w < 14; ++w) {
                uint64_t v = splitmix64(key + 14 * blk + (uint64_t)w);
                for (int j = 0; j < 8; ++j) {
                    int pos = 8 * w + j;
                    if (pos >= 2 && pos < IQ3S_BLOCK_BYTES)
                        o[pos] = (uint8_t)(v >> (8 * j));
                }
            }
            double z = fabs(orc_normal(seed, 2, blk));
            uint16_t h = orc_f32_to_fp16((float)(z * 2e-3));
            o[0] = (uint8_t)(h & 0xff);
            o[1] = (uint8_t)(h >> 8);
        }
}

/* bf16 activations x[i] = bf16(f32(normal(seed, 3, i) * (outlier ? 100 : 1))),
 * outlier iff (rnd(outlier_seed, 4, i) >> 11) < outlier_frac * 2^53. */
void orc_gen_bf16(uint64_t seed, uint64_t outlier_seed, double outlier_frac, int64_t i0, int64_t count,
                  uint16_t *out)
{
    uint64_t thresh = (uint64_t)(outlier_frac * 9007199254740992.0);
    for (int64_t t = 0; t < count; ++t) {
        uint64_t i = (uint64_t)(i0 + t);
        double z = orc_normal(seed, 3, i);
        if (outlier_frac > 0.0 && (orc_rnd(outlier_seed, 4, i) >> 11) < thresh)
            z *= 100.0;
        out[t] = orc_f32_to_bf16((float)z);
    }
}

/* ------------------------------------------------------------ array helpers */
void orc_e4m3_encode_array(const double *in, int64_t n, uint8_t *out)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = orc_e4m3_encode(in[i]);
}

void orc_mxfp8_exponent_array(const float *amax, int64_t n, int32_t *out)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = orc_mxfp8_exponent(amax[i]);
}
