// Shared definitions for the gfx950 kernels of libmambo_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mambo_hip.h"
#include "iq3s_grid.h"

// ----------------------------------------------------------------------------- errors
// Thread-local last error (api.hip). Entry points return a MAMBO_* status.
int mambo_fail(int status, const char *fmt, ...);
int mambo_check_launch(const char *what);
// Records an error that earlier, unrelated HIP work left on the calling thread (taken
// off the thread by the hipGetLastError in MAMBO_LAUNCH); mambo_check_launch then
// reports it through mambo_last_error() (the call itself still succeeds).
void mambo_note_prior_error(hipError_t err);

// Launch with the calling thread's HIP error state taken first, so that the
// mambo_check_launch after it reports this launch's own failure, not one that an
// earlier, unrelated HIP call left behind; that earlier error stays readable through
// mambo_last_error().
#define MAMBO_LAUNCH(...)                                                                          \
    do {                                                                                           \
        mambo_note_prior_error(hipGetLastError());                                                 \
        hipLaunchKernelGGL(__VA_ARGS__);                                                           \
    } while (0)

#define MAMBO_REQUIRE(cond, status, ...)                                                           \
    do {                                                                                           \
        if (!(cond))                                                                               \
            return mambo_fail((status), __VA_ARGS__);                                              \
    } while (0)

// ----------------------------------------------------------------------------- IQ3_S layout
// One IQ3_S super-block: 256 weights in 110 bytes (iq3_s_fp8.py:11-21).
constexpr int kIq3sBlockBytes = 110;
constexpr int kIq3sBlockValues = 256;

// Private tile layout written by mambo_iq3s_prepare/mambo_iq3s_pack and read by the
// projection kernels. One tile = 16 weight rows x one super-block = 1760 bytes,
// tiles ordered [row_tile][block].
//
// The order is the B operand of V_MFMA_SCALE_F32_16X16X128_F8F6F4 over a block's two K
// halves h: lane l (col = l & 15 = row in the tile, q = l >> 4) holds bytes 0-15 at K
// [16q, 16q+16) and bytes 16-31 at K [64+16q, 64+16q+16) of column col, and K block kb
// (K [32kb, 32kb+32), one E8M0 activation scale) of half h holds weight group
// tile_group(kb, h) = {0, 4, 2, 6}[kb] + h. So in half h lane l decodes code slots
// C = 0..7 (slot i = 8h + C of its stream): C < 4 are codes 4(q&1) + C of group
// tile_group(q >> 1, h), C >= 4 codes 4(q&1) + C - 4 of group tile_group(2 + (q >> 1), h).
// Each lane's decoded words are its MFMA operand as they are, with no cross-lane moves.
//   [   0, 1024)  idx stream, bits 0..127 of lane l at 16*l   (dwordx4 per lane)
//   [1024, 1152)  idx stream, bits 128..143 of lane l at 2*l
//   [1152, 1664)  transposed sign words of lane l's halves h = 0, 1 at 8*l + 4h
//   [1664, 1728)  scale byte q (scales[q] of the block: groups 2q, 2q+1) of row col at l
//   [1728, 1760)  fp16 d of row col at 2*col
// idx stream: slot i occupies bits [9i, 9i+9) and holds qs | qh_bit << 8 of its code.
// Transposed sign word P of a half: bit (C + 8j) of P is the sign of weight j of slot C,
// so one rotate places slot C's four signs on bits 7,15,23,31.
// The bytes are a permutation of the 16 source blocks' bytes (16 x 110 = 1760).
__host__ __device__ constexpr int tile_group(int kb, int h) { return ((kb & 1) << 2) + ((kb >> 1) << 1) + h; }
constexpr int kTileRows = 16;
constexpr int kTileBytes = kTileRows * kIq3sBlockBytes;
constexpr int kTileIdxA = 0;
constexpr int kTileIdxB = 1024;
constexpr int kTileSigns = 1152;
constexpr int kTileScales = 1664;
constexpr int kTileD = 1728;
static_assert(kTileD + 2 * kTileRows == kTileBytes, "tile layout must be byte-preserving");

// E4M3 (OCP, bias 7) encodings of the odd grid magnitudes 1,3,...,15 (iq3_s_fp8.py:80-81).
__host__ __device__ constexpr uint32_t e4m3_of_odd(uint32_t m)
{
    return m == 1 ? 0x38u : m == 3 ? 0x44u : m == 5 ? 0x4Au : m == 7 ? 0x4Eu : m == 9 ? 0x51u
         : m == 11 ? 0x53u : m == 13 ? 0x55u : m == 15 ? 0x57u : 0xFFu;
}

struct GridTables {
    uint32_t raw[512];   // magnitudes 1..15 per byte
    uint32_t fp8[512];   // E4M3 bits of the magnitudes (iq3_s_fp8_table)
    uint32_t level[512]; // (magnitude - 1) / 2 per byte: 0..7
};

__host__ __device__ constexpr GridTables make_grid_tables()
{
    GridTables t{{MAMBO_IQ3S_GRID_WORDS}, {}, {}};
    for (int i = 0; i < 512; ++i) {
        uint32_t f = 0, l = 0;
        for (int j = 0; j < 4; ++j) {
            uint32_t m = (t.raw[i] >> (8 * j)) & 0xFFu;
            f |= e4m3_of_odd(m) << (8 * j);
            l |= ((m - 1u) / 2u) << (8 * j);
        }
        t.fp8[i] = f;
        t.level[i] = l;
    }
    return t;
}

inline constexpr GridTables kGridTables = make_grid_tables();

// Exact two-term split of the IQ3_S weight magnitudes for dense FP8 operands. A weight
// is d * (1 + 2s) * (2l + 1) * sign (s: 4-bit group scale, l: 3-bit grid level); the
// integer P = (1 + 2s)(2l + 1) <= 465 needs up to 9 significant bits, E4M3 holds 4.
// P = hi + lo with hi = P rounded to 4 significant bits (ties to even) and lo = P - hi
// (an integer, |lo| <= 16); hi/2 and lo/2 are exact E4M3 values, so an MFMA with B
// scale 2 over both terms gives P exactly. For each s the table holds the E4M3 bytes of
// hi/2 and lo/2 for the eight levels: w[s] = {hi l=0..3, hi l=4..7, lo l=0..3, lo l=4..7},
// byte j of a word = level 4*(word & 1) + j, ready for v_perm_b32 with the level bytes
// of a grid word as selectors.
__host__ __device__ constexpr uint32_t round_to_4_significant_bits(uint32_t p)
{
    int bits = 0;
    while ((p >> bits) != 0u)
        ++bits;
    if (bits <= 4)
        return p;
    const int shift = bits - 4;
    uint32_t q = p >> shift;
    const uint32_t rem = p & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u)))
        ++q;
    return q << shift;
}

// E4M3 bits of k/2 for an integer k whose magnitude has at most 4 significant bits and
// |k| <= 480 (so k/2 is exact in E4M3).
__host__ __device__ constexpr uint32_t e4m3_of_half_integer(int k)
{
    if (k == 0)
        return 0u;
    const uint32_t sign = k < 0 ? 0x80u : 0u;
    const uint32_t a = (uint32_t)(k < 0 ? -k : k);
    int t = 0;
    while ((a >> (t + 1)) != 0u)
        ++t;
    // k/2 = 2^(t-1) * (a / 2^t); E4M3 exponent field t - 1 + 7, mantissa (a*8 >> t) - 8
    return sign | ((uint32_t)(t + 6) << 3) | (((a << 3) >> t) - 8u);
}

struct SplitTables {
    uint32_t w[16][4];
};

__host__ __device__ constexpr SplitTables make_split_tables()
{
    SplitTables t{};
    for (int s = 0; s < 16; ++s)
        for (int l = 0; l < 8; ++l) {
            const uint32_t p = (1u + 2u * s) * (2u * l + 1u);
            const uint32_t hi = round_to_4_significant_bits(p);
            const int lo = (int)p - (int)hi;
            t.w[s][l >> 2] |= e4m3_of_half_integer((int)hi) << (8 * (l & 3));
            t.w[s][2 + (l >> 2)] |= e4m3_of_half_integer(lo) << (8 * (l & 3));
        }
    return t;
}

inline constexpr SplitTables kSplitTables = make_split_tables();

// ----------------------------------------------------------------------------- device helpers
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t funnel_shr(uint32_t hi, uint32_t lo, uint32_t s)
{
    return __builtin_amdgcn_alignbit(hi, lo, s);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h)
{
    _Float16 v = __builtin_bit_cast(_Float16, h);
    return (float)v;
}

// Exact MXFP8 block exponent (quantize_fp8.py:32-38 with an exact ceil(log2(amax/448))):
// amax = m * 2^E, m in [1,2): e = E-8 if m <= 1.75 else E-7; 0 for amax == 0;
// clamped to [-127, 127]. Subnormal amax always gives -127.
__device__ __forceinline__ int mxfp8_exponent(float amax)
{
    uint32_t u = __float_as_uint(amax);
    if (u == 0u)
        return 0;
    if (u < 0x00800000u)
        return -127;
    int E = (int)(u >> 23) - 127;
    int e = ((u & 0x7FFFFFu) <= 0x600000u) ? E - 8 : E - 7;
    return e < -127 ? -127 : e;
}

// |y| <= 448 (or any finite y: saturating) -> E4M3 bits, round to nearest even,
// sign of y kept (including -0). Integer restatement of the OCP conversion.
__device__ __forceinline__ uint32_t e4m3_rne_sw(float y)
{
    uint32_t u = __float_as_uint(y);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7FFFFFFFu;
    uint32_t code;
    if (a < 0x3C800000u) { // < 2^-6: subnormal grid, step 2^-9
        float q = __builtin_rintf(__uint_as_float(a) * 512.0f);
        code = (uint32_t)q; // 0..8; 8 is the smallest normal
    } else {
        uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
        code = (r >> 20) - (120u << 3);
        code = code > 0x7Eu ? 0x7Eu : code;
    }
    return sign | code;
}

// E4M3 rounding path of the quantizer: hardware v_cvt_pk_fp8_f32 (true) or the integer
// restatement e4m3_rne_sw (false). The two agree on every f32 with |x| <= 464 (checked
// on gfx950 over all 2^31 such bit patterns with both signs); the quantizer only feeds
// |x * 2^-e| <= 448.
constexpr bool kQuantHwCvt = true;

// One 32-element MXFP8 group of an unquantized row (bf16 or f32, 16-byte aligned):
// load_group32 reads it as f32 values, quantize_group32 returns its exponent e (the
// E8M0 scale byte is e + 127) and writes the 32 E4M3 codes of x * 2^-e, little-endian
// four per word - the arithmetic of quantize_mxfp8_kernel, so the codes match it.
template <bool kBf16>
__device__ __forceinline__ void load_group32(const void *__restrict__ x, int64_t off, float (&v)[32])
{
    if constexpr (kBf16) {
        const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(x) + off);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 w = p[i];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * i + 2 * j] = __uint_as_float(ws[j] << 16);
                v[8 * i + 2 * j + 1] = __uint_as_float(ws[j] & 0xFFFF0000u);
            }
        }
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(x) + off);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 f = p[i];
            v[4 * i] = f.x;
            v[4 * i + 1] = f.y;
            v[4 * i + 2] = f.z;
            v[4 * i + 3] = f.w;
        }
    }
}

// Four E4M3 codes packed little-endian.
template <bool kHw>
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d)
{
    if constexpr (kHw) {
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
        return (uint32_t)w;
    } else {
        return e4m3_rne_sw(a) | (e4m3_rne_sw(b) << 8) | (e4m3_rne_sw(c) << 16) | (e4m3_rne_sw(d) << 24);
    }
}

// Non-finite inputs (outside the reference's tests: its numpy encoder raises on them and
// its C++ tool rejects them). amax is taken over the magnitude bit patterns as unsigned
// integers, so a NaN beats an infinity and an infinity beats every finite value. A group
// whose amax is not finite gets the E8M0 NaN scale byte 0xFF (the whole group decodes to
// NaN), and each of its codes is the E4M3 NaN 0x7F with the sign of its input.
constexpr uint32_t kNonFiniteBits = 0x7F800000u;
constexpr int kScaleNaN = 0xFF;

__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

// Four E4M3 NaN codes carrying the signs of a..d.
__device__ __forceinline__ uint32_t nan4(float a, float b, float c, float d)
{
    return 0x7F7F7F7Fu | ((__float_as_uint(a) >> 24) & 0x80u) | ((__float_as_uint(b) >> 16) & 0x8000u) |
           ((__float_as_uint(c) >> 8) & 0x800000u) | (__float_as_uint(d) & 0x80000000u);
}

// Returns the E8M0 scale byte (e + 127, or kScaleNaN).
__device__ __forceinline__ int quantize_group32(const float (&v)[32], uint32_t (&codes)[8])
{
    uint32_t amax = 0u;
#pragma unroll
    for (int i = 0; i < 32; ++i)
        amax = max(amax, abs_bits(v[i]));
    if (amax >= kNonFiniteBits) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            codes[i] = nan4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        return kScaleNaN;
    }
    const int e = mxfp8_exponent(__uint_as_float(amax));
#pragma unroll
    for (int i = 0; i < 8; ++i)
        codes[i] = pack4<kQuantHwCvt>(__builtin_ldexpf(v[4 * i], -e), __builtin_ldexpf(v[4 * i + 1], -e),
                                      __builtin_ldexpf(v[4 * i + 2], -e), __builtin_ldexpf(v[4 * i + 3], -e));
    return e + 127;
}

