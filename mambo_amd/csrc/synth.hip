// Counter-based synthetic inputs for benchmarks and full-size checks. Every element is a
// pure function of (seed, stream, index), so any sampled weight row or activation can be
// regenerated independently on the host. Definitions are in include/mambo_hip.h.
#include "mambo_common.h"

namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t stream)
{
    return splitmix64(seed * 0xD1B54A32D192ED03ull + stream);
}

// Irwin-Hall sum of 12 uniforms, exact in double.
__device__ __forceinline__ double normal_at(uint64_t key, uint64_t i)
{
    uint64_t s = 0;
#pragma unroll
    for (int t = 0; t < 12; ++t)
        s += splitmix64(key + 12 * i + (uint64_t)t) >> 32;
    return (double)((int64_t)s - (int64_t)(6ull << 32)) / 4294967296.0;
}

// IEEE binary32 -> binary16, round to nearest even (integer restatement).
__device__ __forceinline__ uint16_t f32_to_fp16_rne(float f)
{
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u)
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    int e = (int)(ax >> 23) - 127;
    uint32_t m = (ax & 0x7FFFFFu) | (ax >= 0x800000u ? 0x800000u : 0u);
    if (ax < 0x800000u)
        e = -126;
    if (e > 15)
        return (uint16_t)(sign | 0x7C00u);
    int shift;
    uint32_t base;
    if (e >= -14) {
        shift = 13;
        base = (uint32_t)(e + 15) << 10;
        m &= 0x7FFFFFu;
    } else {
        shift = 13 + (-14 - e);
        base = 0;
        if (shift > 24)
            return (uint16_t)sign;
    }
    uint32_t qv = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (qv & 1u)))
        qv += 1u;
    return (uint16_t)(sign | (base + qv));
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f)
{
    uint32_t x = __float_as_uint(f);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

// One thread per 110-byte block.
__global__ __launch_bounds__(256) void synth_iq3s_kernel(uint64_t seed, int64_t blocks, int64_t row0, int64_t nrows,
                                                         uint8_t *__restrict__ raw)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrows * blocks)
        return;
    const int64_t r = i / blocks, b = i % blocks;
    const uint64_t blk = (uint64_t)((row0 + r) * blocks + b);
    const uint64_t key1 = stream_key(seed, 1);
    uint8_t *o = raw + i * kIq3sBlockBytes;
    for (int w = 0; w < 14; ++w) {
        const uint64_t v = splitmix64(key1 + 14 * blk + (uint64_t)w);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int pos = 8 * w + j;
            if (pos >= 2 && pos < kIq3sBlockBytes)
                o[pos] = (uint8_t)(v >> (8 * j));
        }
    }
    const double z = fabs(normal_at(stream_key(seed, 2), blk));
    const uint16_t h = f32_to_fp16_rne((float)(z * 2e-3));
    o[0] = (uint8_t)(h & 0xFFu);
    o[1] = (uint8_t)(h >> 8);
}

__global__ __launch_bounds__(256) void synth_bf16_kernel(uint64_t seed, uint64_t outlier_seed, double outlier_frac,
                                                         int64_t i0, int64_t count, uint16_t *__restrict__ out)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= count)
        return;
    const uint64_t i = (uint64_t)(i0 + t);
    double z = normal_at(stream_key(seed, 3), i);
    if (outlier_frac > 0.0) {
        const uint64_t thresh = (uint64_t)(outlier_frac * 9007199254740992.0);
        if ((splitmix64(stream_key(outlier_seed, 4) + i) >> 11) < thresh)
            z *= 100.0;
    }
    out[t] = f32_to_bf16_rne((float)z);
}

} // namespace

extern "C" int mambo_synth_iq3s(uint64_t seed, int64_t blocks, int64_t row0, int64_t nrows, uint8_t *raw,
                                mambo_stream_t stream)
{
    MAMBO_REQUIRE(raw != nullptr && blocks >= 1 && nrows >= 1 && row0 >= 0, MAMBO_ERR_VALUE, "bad arguments");
    const int64_t total = nrows * blocks;
    MAMBO_REQUIRE((total + 255) / 256 <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "too many blocks for one launch");
    MAMBO_LAUNCH(synth_iq3s_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       seed, blocks, row0, nrows, raw);
    return mambo_check_launch("synth_iq3s");
}

extern "C" int mambo_synth_bf16(uint64_t seed, uint64_t outlier_seed, double outlier_frac, int64_t i0, int64_t count,
                                uint16_t *out, mambo_stream_t stream)
{
    MAMBO_REQUIRE(out != nullptr && count >= 1 && i0 >= 0, MAMBO_ERR_VALUE, "bad arguments");
    MAMBO_REQUIRE((count + 255) / 256 <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "count too large for one launch");
    MAMBO_LAUNCH(synth_bf16_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       seed, outlier_seed, outlier_frac, i0, count, out);
    return mambo_check_launch("synth_bf16");
}
