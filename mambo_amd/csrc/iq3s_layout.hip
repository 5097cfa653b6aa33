// IQ3_S weight preparation and the standalone decoder.
//
// prepare: raw GGUF blocks u8[N, B, 110] (any strides and alignment) -> the reference's
// SoA fields (iq3_s_weight.py:25-54: d [B,N], qs [B,N,16], qh [B,N,4], signs [B,N,8],
// scales [B,N]) and/or the private tile layout read by the projection kernels (layout in
// mambo_common.h). One workgroup stages one 16-row x 1-block tile (1760 bytes) in LDS,
// so every field store is a contiguous run.
//
// dequant: SoA fields -> E4M3 bits [N, K] + f32 group scales [N, K/32], the FP8 form of
// decode_iq3_s_blocks (iq3_s_fp8.py:202-222): bits = iq3_s_fp8_table[qs | qh<<8] with
// the sign bits of the group ORed into each byte's bit 7 (iq3_s_fp8.py:105-166), scale
// = f32(d) * (1 + 2*nibble) (iq3_s_fp8.py:186-199).
#include "mambo_common.h"

namespace {

__constant__ GridTables c_grid = kGridTables;

struct RawSrc {
    const uint8_t *raw;
    int64_t sn, sb, sbyte;
};

struct SoaSrc {
    const uint16_t *d;
    const uint32_t *qs;
    const uint16_t *qh;
    const int32_t *signs;
    const uint32_t *scales;
};

// Stage tile (t, b) as 16 rows x 110 bytes in GGUF block order; rows >= n are zero.
__device__ void stage(const RawSrc &s, int64_t n, int64_t blocks, int64_t t, int64_t b,
                      uint8_t (*blk)[112])
{
    for (int i = threadIdx.x; i < kTileRows * kIq3sBlockBytes; i += blockDim.x) {
        int r = i / kIq3sBlockBytes, c = i % kIq3sBlockBytes;
        int64_t row = t * kTileRows + r;
        blk[r][c] = row < n ? s.raw[row * s.sn + b * s.sb + c * s.sbyte] : 0;
    }
    (void)blocks;
}

__device__ void stage(const SoaSrc &s, int64_t n, int64_t blocks, int64_t t, int64_t b,
                      uint8_t (*blk)[112])
{
    (void)blocks;
    // 16 rows x (1 d + 16 qs + 4 qh + 8 signs + 1 scales) = 16 x 30 items
    for (int i = threadIdx.x; i < kTileRows * 30; i += blockDim.x) {
        int r = i / 30, f = i % 30;
        int64_t row = t * kTileRows + r;
        uint8_t *o = blk[r];
        if (row >= n) {
            if (f == 0) {
                for (int c = 0; c < kIq3sBlockBytes; ++c)
                    o[c] = 0;
            }
            continue;
        }
        int64_t e = b * n + row;
        if (f == 0) {
            uint16_t v = s.d[e];
            o[0] = (uint8_t)v;
            o[1] = (uint8_t)(v >> 8);
        } else if (f <= 16) {
            uint32_t v = s.qs[e * 16 + (f - 1)];
            for (int j = 0; j < 4; ++j)
                o[2 + 4 * (f - 1) + j] = (uint8_t)(v >> (8 * j));
        } else if (f <= 20) {
            uint16_t v = s.qh[e * 4 + (f - 17)];
            o[66 + 2 * (f - 17)] = (uint8_t)v;
            o[66 + 2 * (f - 17) + 1] = (uint8_t)(v >> 8);
        } else if (f <= 28) {
            uint32_t v = (uint32_t)s.signs[e * 8 + (f - 21)];
            for (int j = 0; j < 4; ++j)
                o[74 + 4 * (f - 21) + j] = (uint8_t)(v >> (8 * j));
        } else {
            uint32_t v = s.scales[e];
            for (int j = 0; j < 4; ++j)
                o[106 + j] = (uint8_t)(v >> (8 * j));
        }
    }
}

__device__ __forceinline__ uint32_t le32(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Code c (0..63: weights 4c..4c+3 of the block) of slot i (0..15) of lane group q (tile
// layout in mambo_common.h).
__device__ __forceinline__ int slot_code(int q, int i)
{
    const int h = i >> 3, c = i & 7;
    return 8 * tile_group(2 * (c >> 2) + (q >> 1), h) + 4 * (q & 1) + (c & 3);
}

// Transposed sign word of half h of lane group q: bit (C + 8j) = sign of weight j of slot
// 8h + C, i.e. bit 4*code + j of the block's sign bits (bytes 74..105, weight k at bit k).
__device__ __forceinline__ uint32_t half_signs(const uint8_t *o, int q, int h)
{
    uint32_t p = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int code = slot_code(q, 8 * h + c);
        const uint32_t nib = ((uint32_t)o[74 + code / 2] >> (4 * (code & 1))) & 15u;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            p |= ((nib >> j) & 1u) << (c + 8 * j);
    }
    return p;
}

// Write the tile (t, b) in the private layout from the staged blocks.
__device__ void write_tile(uint8_t (*blk)[112], uint8_t *__restrict__ tile)
{
    const int l = threadIdx.x;
    if (l < 64) {
        const int r = l & 15, q = l >> 4;
        const uint8_t *o = blk[r];
        uint32_t w[5] = {0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = slot_code(q, i);
            const uint32_t idx = o[2 + c] | ((((uint32_t)o[66 + c / 8] >> (c % 8)) & 1u) << 8);
            const int p = 9 * i;
            w[p >> 5] |= idx << (p & 31);
            if ((p & 31) > 32 - 9)
                w[(p >> 5) + 1] |= idx >> (32 - (p & 31));
        }
        *reinterpret_cast<uint4 *>(tile + kTileIdxA + 16 * l) = make_uint4(w[0], w[1], w[2], w[3]);
        *reinterpret_cast<uint16_t *>(tile + kTileIdxB + 2 * l) = (uint16_t)w[4];
        *reinterpret_cast<uint2 *>(tile + kTileSigns + 8 * l) = make_uint2(half_signs(o, q, 0), half_signs(o, q, 1));
        tile[kTileScales + l] = o[106 + q];
        if (q == 0) {
            tile[kTileD + 2 * r] = o[0];
            tile[kTileD + 2 * r + 1] = o[1];
        }
    }
}

template <class Src>
__global__ __launch_bounds__(256) void prepare_kernel(Src src, int64_t n, int64_t blocks,
                                                      uint16_t *__restrict__ d, uint32_t *__restrict__ qs,
                                                      uint16_t *__restrict__ qh, int32_t *__restrict__ signs,
                                                      uint32_t *__restrict__ scales, uint8_t *__restrict__ packed)
{
    __shared__ uint8_t blk[kTileRows][112];
    const int64_t t = blockIdx.x;
    for (int64_t b = blockIdx.y; b < blocks; b += gridDim.y) {
        __syncthreads();
        stage(src, n, blocks, t, b, blk);
        __syncthreads();
        const int i = threadIdx.x;
        const int r = i >> 4, w = i & 15; // 16 rows x 16 words
        const int64_t row = t * kTileRows + r;
        if (row < n) {
            const int64_t e = b * n + row;
            const uint8_t *o = blk[r];
            if (qs)
                qs[e * 16 + w] = le32(o + 2 + 4 * w);
            if (signs && w < 8)
                signs[e * 8 + w] = (int32_t)le32(o + 74 + 4 * w);
            if (qh && w < 4)
                qh[e * 4 + w] = (uint16_t)(o[66 + 2 * w] | (o[67 + 2 * w] << 8));
            if (w == 0) {
                if (d)
                    d[e] = (uint16_t)(o[0] | (o[1] << 8));
                if (scales)
                    scales[e] = le32(o + 106);
            }
        }
        if (packed)
            write_tile(blk, packed + (t * blocks + b) * (int64_t)kTileBytes);
    }
}

__global__ __launch_bounds__(256) void dequant_kernel(const uint16_t *__restrict__ d, const uint32_t *__restrict__ qs,
                                                      const uint16_t *__restrict__ qh,
                                                      const int32_t *__restrict__ signs,
                                                      const uint32_t *__restrict__ scales, int64_t n,
                                                      int64_t blocks, uint8_t *__restrict__ values,
                                                      float *__restrict__ out_scales)
{
    __shared__ uint32_t lut[512];
    for (int i = threadIdx.x; i < 512; i += blockDim.x)
        lut[i] = c_grid.fp8[i];
    __syncthreads();
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = n * blocks * 8;
    if (gid >= total)
        return;
    const int g = (int)(gid & 7);
    const int64_t b = (gid >> 3) % blocks;
    const int64_t row = (gid >> 3) / blocks;
    const int64_t e = b * n + row;
    const uint32_t q0 = qs[e * 16 + 2 * g], q1 = qs[e * 16 + 2 * g + 1];
    const uint32_t hb = reinterpret_cast<const uint8_t *>(qh)[e * 8 + g];
    const uint32_t sw = (uint32_t)signs[e * 8 + g];
    const uint32_t s = (scales[e] >> (4 * g)) & 15u;
    uint32_t out[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t lo = ((c < 4 ? q0 : q1) >> (8 * (c & 3))) & 0xFFu;
        const uint32_t idx = lo | (((hb >> c) & 1u) << 8);
        const uint32_t nib = (sw >> (4 * c)) & 15u;
        const uint32_t mask = ((nib & 1u) << 7) | ((nib & 2u) << 14) | ((nib & 4u) << 21) | ((nib & 8u) << 28);
        out[c] = lut[idx] | mask;
    }
    uint4 *vp = reinterpret_cast<uint4 *>(values + row * blocks * 256 + b * 256 + 32 * g);
    vp[0] = make_uint4(out[0], out[1], out[2], out[3]);
    vp[1] = make_uint4(out[4], out[5], out[6], out[7]);
    out_scales[row * blocks * 8 + b * 8 + g] = half_bits_to_float(d[e]) * (float)(1u + 2u * s);
}

} // namespace

extern "C" int64_t mambo_iq3s_packed_bytes(int64_t n, int64_t blocks)
{
    if (n < 1 || blocks < 1)
        return 0;
    return ((n + kTileRows - 1) / kTileRows) * blocks * (int64_t)kTileBytes;
}

template <class Src>
static int launch_prepare(const Src &src, int64_t n, int64_t blocks, uint16_t *d, uint32_t *qs, uint16_t *qh,
                          int32_t *signs, uint32_t *scales, uint8_t *packed, hipStream_t stream)
{
    const int64_t tiles = (n + kTileRows - 1) / kTileRows;
    MAMBO_REQUIRE(tiles <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "N too large");
    dim3 grid((unsigned)tiles, (unsigned)(blocks < 65535 ? blocks : 65535));
    MAMBO_LAUNCH(prepare_kernel<Src>, grid, dim3(256), 0, stream, src, n, blocks, d, qs, qh, signs, scales,
                       packed);
    return mambo_check_launch("iq3s_prepare");
}

extern "C" int mambo_iq3s_prepare(const uint8_t *raw, int64_t n, int64_t blocks, int64_t stride_n,
                                  int64_t stride_b, int64_t stride_byte, uint16_t *d, uint32_t *qs,
                                  uint16_t *qh, int32_t *signs, uint32_t *scales, uint8_t *packed,
                                  mambo_stream_t stream)
{
    MAMBO_REQUIRE(raw != nullptr, MAMBO_ERR_VALUE, "raw must not be NULL");
    MAMBO_REQUIRE(n >= 1 && blocks >= 1, MAMBO_ERR_VALUE, "IQ3_S weight must have positive N and K");
    MAMBO_REQUIRE(d || qs || qh || signs || scales || packed, MAMBO_ERR_VALUE, "no output requested");
    MAMBO_REQUIRE(((uintptr_t)qs % 4 == 0) && ((uintptr_t)signs % 4 == 0) && ((uintptr_t)scales % 4 == 0) &&
                      ((uintptr_t)d % 2 == 0) && ((uintptr_t)qh % 2 == 0) && ((uintptr_t)packed % 16 == 0),
                  MAMBO_ERR_VALUE, "SoA fields must be naturally aligned and packed 16-byte aligned");
    RawSrc src{raw, stride_n, stride_b, stride_byte};
    return launch_prepare(src, n, blocks, d, qs, qh, signs, scales, packed, (hipStream_t)stream);
}

extern "C" int mambo_iq3s_pack(const uint16_t *d, const uint32_t *qs, const uint16_t *qh, const int32_t *signs,
                               const uint32_t *scales, int64_t n, int64_t blocks, uint8_t *packed,
                               mambo_stream_t stream)
{
    MAMBO_REQUIRE(d && qs && qh && signs && scales && packed, MAMBO_ERR_VALUE, "null pointer");
    MAMBO_REQUIRE(n >= 1 && blocks >= 1, MAMBO_ERR_VALUE, "IQ3_S weight must have positive N and K");
    MAMBO_REQUIRE((uintptr_t)packed % 16 == 0, MAMBO_ERR_VALUE, "packed must be 16-byte aligned");
    SoaSrc src{d, qs, qh, signs, scales};
    return launch_prepare(src, n, blocks, nullptr, nullptr, nullptr, nullptr, nullptr, packed,
                          (hipStream_t)stream);
}

extern "C" int mambo_iq3s_dequant(const uint16_t *d, const uint32_t *qs, const uint16_t *qh, const int32_t *signs,
                                  const uint32_t *scales, int64_t n, int64_t blocks, uint8_t *values,
                                  float *out_scales, mambo_stream_t stream)
{
    MAMBO_REQUIRE(d && qs && qh && signs && scales && values && out_scales, MAMBO_ERR_VALUE, "null pointer");
    MAMBO_REQUIRE(n >= 1 && blocks >= 1, MAMBO_ERR_VALUE, "IQ3_S weight must have positive N and K");
    MAMBO_REQUIRE((uintptr_t)values % 16 == 0, MAMBO_ERR_VALUE, "values must be 16-byte aligned");
    const int64_t total = n * blocks * 8;
    MAMBO_REQUIRE((total + 255) / 256 <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "weight too large");
    MAMBO_LAUNCH(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, d,
                       qs, qh, signs, scales, n, blocks, values, out_scales);
    return mambo_check_launch("iq3s_dequant");
}
