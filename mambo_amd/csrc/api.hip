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

int mambo_check_launch(const char *what)
{
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return mambo_fail(MAMBO_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(err));
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
    hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)src, (uint4 *)dst, n16);
    return mambo_check_launch("copy_bytes");
}

extern "C" int mambo_fill_f32(float *ptr, int64_t n, float value, mambo_stream_t stream)
{
    MAMBO_REQUIRE(n >= 0, MAMBO_ERR_VALUE, "n must be >= 0");
    if (n == 0)
        return MAMBO_OK;
    MAMBO_REQUIRE(ptr != nullptr, MAMBO_ERR_VALUE, "ptr must not be NULL");
    int64_t blocks = (n + 1023) / 1024;
    MAMBO_REQUIRE(blocks <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "n too large");
    hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, ptr, n, value);
    return mambo_check_launch("fill_f32");
}
