// Error state, build information, codebook export and small utility kernels.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "mambo_common.h"

static thread_local char g_last_error[1024] = "";

int mambo_fail(int status, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

// An error found on the thread before one of this call's launches (hipSuccess: none).
static thread_local hipError_t g_prior_error = hipSuccess;

void mambo_note_prior_error(hipError_t err)
{
    if (err != hipSuccess && g_prior_error == hipSuccess)
        g_prior_error = err;
}

int mambo_check_launch(const char *what)
{
    const hipError_t prior = g_prior_error;
    g_prior_error = hipSuccess;
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return mambo_fail(MAMBO_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(err));
    if (prior != hipSuccess) // the call succeeded; keep the earlier error readable
        return mambo_fail(MAMBO_OK, "%s: ok; an earlier HIP error left on this thread was taken off it before "
                                    "the launch: %s", what, hipGetErrorString(prior));
    g_last_error[0] = '\0';
    return MAMBO_OK;
}

extern "C" const char *mambo_last_error(void) { return g_last_error; }

extern "C" int mambo_abi_version(void) { return 100; }

extern "C" const char *mambo_build_arch(void) { return "gfx950"; }

extern "C" int mambo_device_arch(int device, char *buf, int buf_len)
{
    MAMBO_REQUIRE(buf != nullptr && buf_len > 0, MAMBO_ERR_VALUE, "buf must be a non-empty buffer");
    hipDeviceProp_t prop;
    hipError_t err = hipGetDeviceProperties(&prop, device);
    if (err != hipSuccess)
        return mambo_fail(MAMBO_ERR_RUNTIME, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(err));
    snprintf(buf, (size_t)buf_len, "%s", prop.gcnArchName);
    return MAMBO_OK;
}

extern "C" int mambo_iq3s_grid(uint32_t *out)
{
    MAMBO_REQUIRE(out != nullptr, MAMBO_ERR_VALUE, "out must not be NULL");
    memcpy(out, kGridTables.raw, sizeof(kGridTables.raw));
    return MAMBO_OK;
}

extern "C" int mambo_iq3s_fp8_grid(uint32_t *out)
{
    MAMBO_REQUIRE(out != nullptr, MAMBO_ERR_VALUE, "out must not be NULL");
    memcpy(out, kGridTables.fp8, sizeof(kGridTables.fp8));
    return MAMBO_OK;
}

extern "C" int mambo_iq3s_split_table(uint32_t *out)
{
    MAMBO_REQUIRE(out != nullptr, MAMBO_ERR_VALUE, "out must not be NULL");
    for (int s = 0; s < 16; ++s)
        for (int w = 0; w < 4; ++w)
            out[4 * s + w] = kSplitTables.w[s][w];
    return MAMBO_OK;
}

__global__ void fill_f32_kernel(float *__restrict__ p, int64_t n, float v)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x * 4 + threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j, i += blockDim.x)
        if (i < n)
            p[i] = v;
}

__global__ void copy_bytes_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst, int64_t n16)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

extern "C" int mambo_copy_bytes(const void *src, void *dst, int64_t bytes, mambo_stream_t stream)
{
    MAMBO_REQUIRE(bytes >= 0 && bytes % 16 == 0, MAMBO_ERR_VALUE, "bytes must be a non-negative multiple of 16");
    if (bytes == 0)
        return MAMBO_OK;
    MAMBO_REQUIRE(src && dst && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0, MAMBO_ERR_VALUE,
                  "src and dst must be non-NULL and 16-byte aligned");
    const int64_t n16 = bytes / 16;
    const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, 4096);
    MAMBO_LAUNCH(copy_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)src, (uint4 *)dst, n16);
    return mambo_check_launch("copy_bytes");
}

// Plain read: each thread XORs the 16-byte chunks i, i + stride, ... and writes its XOR
// to sink[thread]. Grid of kReadWorkgroups x 256. One load per iteration: at any moment
// the grid reads one contiguous span (measured 6.5 TB/s on 1 GB; four strided loads per
// iteration measured 5.6 TB/s).
constexpr int64_t kReadWorkgroups = MAMBO_READ_SINK_WORDS / 256;

__global__ __launch_bounds__(256) void read_bytes_kernel(const uint4 *__restrict__ src, int64_t n16,
                                                         uint32_t *__restrict__ sink)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t x = 0;
    for (int64_t i = t; i < n16; i += stride) {
        const uint4 v = src[i];
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    sink[t] = x;
}

extern "C" int mambo_read_bytes(const void *src, int64_t bytes, uint32_t *sink, mambo_stream_t stream)
{
    MAMBO_REQUIRE(bytes >= 0 && bytes % 16 == 0, MAMBO_ERR_VALUE, "bytes must be a non-negative multiple of 16");
    MAMBO_REQUIRE(sink != nullptr, MAMBO_ERR_VALUE, "sink must not be NULL");
    MAMBO_REQUIRE(bytes == 0 || (src != nullptr && (uintptr_t)src % 16 == 0), MAMBO_ERR_VALUE,
                  "src must be non-NULL and 16-byte aligned");
    MAMBO_LAUNCH(read_bytes_kernel, dim3((unsigned)kReadWorkgroups), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)src, bytes / 16, sink);
    return mambo_check_launch("read_bytes");
}

// Scaled-MFMA throughput: every wave runs `iters` rounds of eight independent chains of
// v_mfma_scale_f32_16x16x128_f8f6f4 on E4M3 1.0 operands with unit E8M0 scales (each
// MFMA adds 128 to every accumulator element), then writes the sum of its 32
// accumulator values per lane: 8 * 4 * 128 * iters.
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float *__restrict__ out)
{
    const v8i one = {0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838};
    v4f c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        c[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            c[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(one, one, c[j], 0, 0, 0, 127, 0, 127);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        s += (c[j][0] + c[j][1]) + (c[j][2] + c[j][3]);
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

extern "C" int mambo_mfma_peak(int64_t workgroups, int iters, float *out, mambo_stream_t stream)
{
    MAMBO_REQUIRE(workgroups >= 1 && workgroups <= 65536, MAMBO_ERR_VALUE, "workgroups must be in [1, 65536]");
    MAMBO_REQUIRE(iters >= 0 && iters <= (1 << 20), MAMBO_ERR_VALUE, "iters must be in [0, 2^20]");
    MAMBO_REQUIRE(out != nullptr, MAMBO_ERR_VALUE, "out must not be NULL");
    MAMBO_LAUNCH(mfma_peak_kernel, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream, iters, out);
    return mambo_check_launch("mfma_peak");
}

extern "C" int mambo_fill_f32(float *ptr, int64_t n, float value, mambo_stream_t stream)
{
    MAMBO_REQUIRE(n >= 0, MAMBO_ERR_VALUE, "n must be >= 0");
    if (n == 0)
        return MAMBO_OK;
    MAMBO_REQUIRE(ptr != nullptr, MAMBO_ERR_VALUE, "ptr must not be NULL");
    int64_t blocks = (n + 1023) / 1024;
    MAMBO_REQUIRE(blocks <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "n too large");
    MAMBO_LAUNCH(fill_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, ptr, n, value);
    return mambo_check_launch("fill_f32");
}
