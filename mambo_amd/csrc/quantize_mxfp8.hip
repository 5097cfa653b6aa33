// MXFP8 activation quantizer for gfx950.
//
// Semantics follow the reference kernel quantize_fp8_group / quantize_activation_fp8
// (src/python/mambo/kernels/quantize_fp8.py:23-52): per 32 consecutive K elements of a
// row, amax -> e = max(ceil(log2(amax/448)), -127) (e = 0 when amax == 0), one E8M0
// scale byte e+127 and 32 E4M3 codes of x * 2^-e rounded to nearest even. The exponent
// is computed exactly from the bits of amax instead of through f32 log2. A group holding
// a NaN or an infinity gets scale byte 0xFF and E4M3 NaN codes (quantize_group32).
//
// Mapping: four lanes per 32-element group, eight elements per lane, so every
// wave-wide load and store instruction covers one contiguous span (bf16: 1 KiB per
// load). amax is reduced across the quad with two lane swaps. The kernel is HBM-bound:
// M*K*(in_bytes + 1 + 1/32) bytes per call.
#include "mambo_common.h"

namespace {


// Rows per workgroup iteration: the loads of both rows are issued before either is
// converted, two 16-byte loads in flight per lane ([4096,4096] bf16: 4345 -> 4565 GB/s;
// 4 and 8 rows, with a quarter / eighth of the workgroups, measured 6% and 16% slower).
constexpr int kQuantRows = 2;

// The input is read once and the codes written once: both go through with the
// non-temporal hint (bf16 [4096,4096] from a HIP graph: 3.89 -> 4.34 TB/s).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool kBf16>
__device__ __forceinline__ void load8(const void *__restrict__ x, int64_t off, float v[8])
{
    if constexpr (kBf16) {
        const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(x) + off));
        uint32_t w[4] = {r[0], r[1], r[2], r[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    } else {
        const f32x4 *p = reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(x) + off);
        const f32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
        v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    }
}

template <bool kBf16>
__device__ __forceinline__ void load8_scalar(const void *__restrict__ x, int64_t off, float v[8])
{
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if constexpr (kBf16)
            v[i] = __uint_as_float((uint32_t)(reinterpret_cast<const uint16_t *>(x)[off + i]) << 16);
        else
            v[i] = reinterpret_cast<const float *>(x)[off + i];
    }
}

template <bool kBf16, bool kVec, bool kHw>
__global__ __launch_bounds__(256) void quantize_mxfp8_kernel(const void *__restrict__ x, int64_t ldx,
                                                             int64_t m, int64_t groups,
                                                             uint8_t *__restrict__ values, int64_t ldv,
                                                             uint8_t *__restrict__ scales, int64_t lds)
{
    const int64_t g = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 2);
    const int j = threadIdx.x & 3;
    const bool ok = g < groups;
    constexpr int R = kQuantRows;
    for (int64_t row0 = (int64_t)blockIdx.y * R; row0 < m; row0 += (int64_t)gridDim.y * R) {
        float v[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (ok && row0 + r < m) {
                const int64_t off = (row0 + r) * ldx + 32 * g + 8 * j;
                if constexpr (kVec)
                    load8<kBf16>(x, off, v[r]);
                else
                    load8_scalar<kBf16>(x, off, v[r]);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    v[r][i] = 0.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = row0 + r;
            // amax over the magnitude bit patterns (NaN > inf > finite; see quantize_group32)
            uint32_t amax = 0u;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                amax = max(amax, abs_bits(v[r][i]));
            amax = max(amax, (uint32_t)__shfl_xor((int)amax, 1));
            amax = max(amax, (uint32_t)__shfl_xor((int)amax, 2));
            const bool finite = amax < kNonFiniteBits;
            const int e = finite ? mxfp8_exponent(__uint_as_float(amax)) : 0;
            if (ok && row < m) {
                float y[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    y[i] = __builtin_ldexpf(v[r][i], -e); // exact scaling by a power of two
                uint2 out;
                if (finite) {
                    out.x = pack4<kHw>(y[0], y[1], y[2], y[3]);
                    out.y = pack4<kHw>(y[4], y[5], y[6], y[7]);
                } else {
                    out.x = nan4(y[0], y[1], y[2], y[3]);
                    out.y = nan4(y[4], y[5], y[6], y[7]);
                }
                uint8_t *vp = values + row * ldv + 32 * g + 8 * j;
                if constexpr (kVec) {
                    __builtin_nontemporal_store(u32x2{out.x, out.y}, reinterpret_cast<u32x2 *>(vp));
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        vp[i] = (uint8_t)(out.x >> (8 * i));
                        vp[4 + i] = (uint8_t)(out.y >> (8 * i));
                    }
                }
                if (j == 0)
                    scales[row * lds + g] = (uint8_t)(finite ? e + 127 : kScaleNaN);
            }
        }
    }
}

__global__ void e4m3_convert_kernel(const float *__restrict__ in, int64_t n, uint8_t *__restrict__ sw,
                                    uint8_t *__restrict__ hw)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n)
        return;
    float v = in[i];
    if (sw)
        sw[i] = (uint8_t)e4m3_rne_sw(v);
    if (hw)
        hw[i] = (uint8_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false);
}

template <bool kBf16, bool kVec>
int launch(const void *x, int64_t m, int64_t groups, int64_t ldx, uint8_t *values, int64_t ldv,
           uint8_t *scales, int64_t lds, hipStream_t stream)
{
    const int64_t ry = (m + kQuantRows - 1) / kQuantRows;
    dim3 grid((unsigned)((groups + 63) / 64), (unsigned)(ry < 65535 ? ry : 65535));
    MAMBO_LAUNCH((quantize_mxfp8_kernel<kBf16, kVec, kQuantHwCvt>), grid, dim3(256), 0, stream,
                       x, ldx, m, groups, values, ldv, scales, lds);
    return mambo_check_launch("quantize_mxfp8");
}

} // namespace

extern "C" int mambo_quantize_mxfp8(const void *x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                                    uint8_t *values, int64_t ldv, uint8_t *scales, int64_t lds,
                                    mambo_stream_t stream)
{
    MAMBO_REQUIRE(x_dtype == MAMBO_DTYPE_F32 || x_dtype == MAMBO_DTYPE_BF16, MAMBO_ERR_VALUE,
                  "activation dtype must be float32 or bfloat16");
    MAMBO_REQUIRE(m >= 1 && k >= 32 && k % 32 == 0, MAMBO_ERR_VALUE,
                  "activation must be [M,K] with M >= 1 and K divisible by 32 (got M=%lld K=%lld)",
                  (long long)m, (long long)k);
    MAMBO_REQUIRE(ldx >= k && ldv >= k && lds >= k / 32, MAMBO_ERR_VALUE, "row strides must cover K");
    MAMBO_REQUIRE(x && values && scales, MAMBO_ERR_VALUE, "null pointer");
    const int64_t groups = k / 32;
    MAMBO_REQUIRE((groups + 63) / 64 <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "K too large");
    const size_t esz = x_dtype == MAMBO_DTYPE_BF16 ? 2 : 4;
    const bool vec = ((uintptr_t)x % 16 == 0) && ((ldx * (int64_t)esz) % 16 == 0) &&
                     ((uintptr_t)values % 8 == 0) && (ldv % 8 == 0);
    hipStream_t s = (hipStream_t)stream;
    if (x_dtype == MAMBO_DTYPE_BF16)
        return vec ? launch<true, true>(x, m, groups, ldx, values, ldv, scales, lds, s)
                   : launch<true, false>(x, m, groups, ldx, values, ldv, scales, lds, s);
    return vec ? launch<false, true>(x, m, groups, ldx, values, ldv, scales, lds, s)
               : launch<false, false>(x, m, groups, ldx, values, ldv, scales, lds, s);
}

extern "C" int mambo_e4m3_convert(const float *in, int64_t n, uint8_t *out_sw, uint8_t *out_hw,
                                  mambo_stream_t stream)
{
    MAMBO_REQUIRE(n >= 0 && in != nullptr, MAMBO_ERR_VALUE, "bad input");
    if (n == 0)
        return MAMBO_OK;
    MAMBO_LAUNCH(e4m3_convert_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       in, n, out_sw, out_hw);
    return mambo_check_launch("e4m3_convert");
}
