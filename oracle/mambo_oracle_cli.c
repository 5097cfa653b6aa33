/*
 * Command-line front end of the CPU oracle (TEST INFRASTRUCTURE ONLY; see
 * mambo_oracle.c). It speaks the protocol of the reference's oracle executable,
 * tests/cpp/reference/ggml_reference.cpp:
 *
 *   mambo_oracle_cli --op matmul --model PATH --weight TENSOR --m M
 *                    [--dequant-rows N] [--benchmark] [--benchmark-iters N]
 *
 * stdin: exactly M*K little-endian float32 values, row-major [M, K] (a short or long
 * input is an error, as are NaN and infinity: ggml_reference.cpp:143-164,458-460).
 * stdout: four NumPy .npy arrays (ggml_reference.cpp:232-268): a u8 array holding the
 * JSON metadata, then f32 dequant_rows [N', K], ggml_dequant_f64 [M, N] and
 * mxfp8_f64 [M, N]. The first two are the reference's CPU path (to_float of each IQ3_S
 * row, float64-accumulated dot, cast to f32: ggml_reference.cpp:495-523). The
 * reference's third array comes from ggml's CUDA backend, which quantizes activations
 * to Q8_1 and is not part of this path; in its place mxfp8_f64 is what the MI355X path
 * computes: the activations MXFP8-quantized (quantize_fp8.py:23-39), then the same
 * float64 dot with the decoded weights.
 * --benchmark: nothing on stdout; one line on stderr (ggml_reference.cpp:317-343):
 *   benchmark backend=cpu op=matmul m= n= k= warmup=5 iterations= mean_us= batched_us=
 *   event_us=
 * timing the mxfp8_f64 computation (quantize + decode + dot) on the CPU. mean_us times
 * each iteration alone, batched_us all of them together; a CPU has no device events,
 * so event_us is the process CPU time per iteration divided by the OpenMP threads.
 * Errors: "mambo_oracle_cli: <message>" on stderr, exit 1.
 */
#include <errno.h>
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* mambo_oracle.c */
void orc_dequant_iq3s(const uint8_t *raw, int64_t n, int64_t nb, float *out);
void orc_quantize_mxfp8_f32(const float *x, int64_t m, int64_t k, int64_t ldx, uint8_t *values, uint8_t *scales);
void orc_mxfp8_decode(const uint8_t *values, const uint8_t *scales, int64_t m, int64_t k, float *out);

#define GGML_TYPE_IQ3_S 21
#define IQ3S_BLOCK_BYTES 110
#define IQ3S_BLOCK_VALUES 256

static void die(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    fputs("mambo_oracle_cli: ", stderr);
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    va_end(ap);
    exit(1);
}

/* ------------------------------------------------------------------ GGUF reader
 * GGUF v2/v3 (little-endian): magic, u32 version, u64 tensor count, u64 metadata
 * count, metadata (u64-length key, u32 type, value), tensor records (name, u32 n_dims,
 * u64 ne[n_dims], u32 ggml type, u64 offset relative to the data section), data
 * section at the header end rounded up to general.alignment (default 32). */
typedef struct {
    FILE *f;
    const char *path;
} Reader;

static void rd(Reader *r, void *dst, size_t n, const char *what)
{
    if (fread(dst, 1, n, r->f) != n)
        die("truncated GGUF file %s while reading %s", r->path, what);
}

static uint64_t rd_u64(Reader *r, const char *what)
{
    uint64_t v;
    rd(r, &v, 8, what);
    return v;
}

static uint32_t rd_u32(Reader *r, const char *what)
{
    uint32_t v;
    rd(r, &v, 4, what);
    return v;
}

/* a GGUF string; returns a malloc'd NUL-terminated copy */
static char *rd_str(Reader *r, const char *what)
{
    uint64_t n = rd_u64(r, what);
    if (n > (1u << 20))
        die("GGUF %s is unreasonably long (%llu bytes)", what, (unsigned long long)n);
    char *s = (char *)malloc(n + 1);
    rd(r, s, (size_t)n, what);
    s[n] = '\0';
    return s;
}

static int meta_size(uint32_t type)
{
    static const int sizes[13] = {1, 1, 2, 2, 4, 4, 4, 1, -1, -1, 8, 8, 8};
    return type < 13 ? sizes[type] : -2;
}

/* Skips one metadata value; returns it when it is an unsigned/signed integer (for
 * general.alignment), else -1. */
static int64_t skip_value(Reader *r, uint32_t type, const char *key)
{
    int size = meta_size(type);
    if (size == -2)
        die("GGUF metadata %s has unknown type %u", key, type);
    if (type == 8) {
        free(rd_str(r, key));
        return -1;
    }
    if (type == 9) {
        uint32_t elem = rd_u32(r, key);
        uint64_t count = rd_u64(r, key);
        int esize = meta_size(elem);
        if (elem == 9 || esize == -2)
            die("GGUF metadata %s has an unsupported array element type %u", key, elem);
        for (uint64_t i = 0; i < count; ++i) {
            if (elem == 8)
                free(rd_str(r, key));
            else if (fseek(r->f, esize, SEEK_CUR) != 0)
                die("truncated GGUF file %s", r->path);
        }
        return -1;
    }
    uint8_t raw[8] = {0};
    rd(r, raw, (size_t)size, key);
    switch (type) {
    case 0: return raw[0];
    case 2: return (int64_t)(raw[0] | raw[1] << 8);
    case 4: return (int64_t)((uint32_t)raw[0] | (uint32_t)raw[1] << 8 | (uint32_t)raw[2] << 16 | (uint32_t)raw[3] << 24);
    case 10: {
        uint64_t v;
        memcpy(&v, raw, 8);
        return v > INT64_MAX ? -1 : (int64_t)v;
    }
    default: return -1;
    }
}

typedef struct {
    int64_t k, n;
    uint64_t offset, bytes, row_bytes;
    uint32_t type;
} TensorInfo;

static TensorInfo find_tensor(const char *path, const char *name)
{
    Reader r = {fopen(path, "rb"), path};
    if (!r.f)
        die("cannot open GGUF model %s: %s", path, strerror(errno));
    char magic[4];
    rd(&r, magic, 4, "magic");
    if (memcmp(magic, "GGUF", 4) != 0)
        die("%s is not a GGUF file", path);
    uint32_t version = rd_u32(&r, "version");
    if (version != 2 && version != 3)
        die("unsupported GGUF version %u", version);
    uint64_t n_tensors = rd_u64(&r, "tensor count"), n_meta = rd_u64(&r, "metadata count");
    if (n_tensors > 10000000 || n_meta > 10000000)
        die("unreasonable GGUF header counts");
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_meta; ++i) {
        char *key = rd_str(&r, "metadata key");
        uint32_t type = rd_u32(&r, "metadata type");
        int64_t v = skip_value(&r, type, key);
        if (strcmp(key, "general.alignment") == 0) {
            if (v <= 0 || (v & (v - 1)))
                die("GGUF general.alignment must be a positive power of two");
            alignment = (uint64_t)v;
        }
        free(key);
    }
    TensorInfo found = {0};
    int have = 0;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        char *tname = rd_str(&r, "tensor name");
        uint32_t n_dims = rd_u32(&r, "tensor dimension count");
        if (n_dims < 1 || n_dims > 4)
            die("tensor %s has unsupported dimension count %u", tname, n_dims);
        uint64_t ne[4] = {1, 1, 1, 1};
        for (uint32_t d = 0; d < n_dims; ++d)
            ne[d] = rd_u64(&r, "tensor dims");
        uint32_t type = rd_u32(&r, "tensor type");
        uint64_t rel = rd_u64(&r, "tensor offset");
        if (strcmp(tname, name) == 0) {
            if (type != GGML_TYPE_IQ3_S)
                die("unsupported ggml tensor type for matmul: type %u (currently supported type: iq3_s)", type);
            if (ne[0] == 0 || ne[1] == 0 || ne[2] != 1 || ne[3] != 1 || ne[0] > INT32_MAX || ne[1] > INT32_MAX)
                die("tensor must be a nonempty rank-2 GGUF tensor");
            if (ne[0] % IQ3S_BLOCK_VALUES)
                die("IQ3_S tensor row width is not divisible by the quantization block size");
            found.k = (int64_t)ne[0];
            found.n = (int64_t)ne[1];
            found.type = type;
            found.row_bytes = ne[0] / IQ3S_BLOCK_VALUES * IQ3S_BLOCK_BYTES;
            found.bytes = found.row_bytes * ne[1];
            found.offset = rel;
            have = 1;
        }
        free(tname);
    }
    if (!have)
        die("tensor not found in GGUF: %s", name);
    long pos = ftell(r.f);
    uint64_t data = ((uint64_t)pos + alignment - 1) / alignment * alignment;
    if (found.offset % alignment)
        die("tensor offset is not aligned to %llu", (unsigned long long)alignment);
    found.offset += data;
    if (fseek(r.f, 0, SEEK_END) != 0)
        die("cannot seek in %s", path);
    uint64_t size = (uint64_t)ftell(r.f);
    fclose(r.f);
    if (found.offset > size || found.bytes > size - found.offset)
        die("tensor data range extends past the GGUF file size");
    return found;
}

/* ------------------------------------------------------------------ NumPy output */
static void write_all(const void *p, size_t n, const char *what)
{
    if (fwrite(p, 1, n, stdout) != n)
        die("failed while writing %s to stdout", what);
}

static void npy_header(const char *descr, const char *shape)
{
    char header[256];
    int len = snprintf(header, sizeof header, "{'descr': '%s', 'fortran_order': False, 'shape': %s, }", descr, shape);
    /* pad with spaces so that magic + version + length + header (with the newline) is a
     * multiple of 16 */
    int total = 10 + len + 1;
    int pad = (16 - total % 16) % 16;
    for (int i = 0; i < pad; ++i)
        header[len++] = ' ';
    header[len++] = '\n';
    const uint8_t pre[10] = {0x93, 'N', 'U', 'M', 'P', 'Y', 1, 0, (uint8_t)(len & 0xFF), (uint8_t)(len >> 8)};
    write_all(pre, 10, "NumPy magic");
    write_all(header, (size_t)len, "NumPy header");
}

static void npy_f32(const float *v, int64_t rows, int64_t cols)
{
    char shape[64];
    snprintf(shape, sizeof shape, "(%lld, %lld)", (long long)rows, (long long)cols);
    npy_header("<f4", shape);
    write_all(v, sizeof(float) * (size_t)(rows * cols), "NumPy array");
}

/* ------------------------------------------------------------------ arguments */
static uint64_t parse_count(const char *text, const char *name, int allow_zero)
{
    char *end = NULL;
    errno = 0;
    if (!*text || *text == '-' || *text == '+')
        die(allow_zero ? "%s must be a nonnegative integer" : "%s must be a positive integer", name);
    unsigned long long v = strtoull(text, &end, 10);
    if (errno || *end || (!allow_zero && v == 0))
        die(allow_zero ? "%s must be a nonnegative integer" : "%s must be a positive integer", name);
    return v;
}

static double now_us(clockid_t clock)
{
    struct timespec t;
    clock_gettime(clock, &t);
    return (double)t.tv_sec * 1e6 + (double)t.tv_nsec * 1e-3;
}

/* out[i, j] = f32(sum_t f64(w[j, t]) * f64(x[i, t])) over all weight rows */
static void dot_f64(const float *x, int64_t m, int64_t k, const float *w, int64_t n, float *out)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t j = 0; j < n; ++j)
        for (int64_t i = 0; i < m; ++i) {
            double acc = 0.0;
            const float *wr = w + j * k, *xr = x + i * k;
            for (int64_t t = 0; t < k; ++t)
                acc += (double)wr[t] * (double)xr[t];
            out[i * n + j] = (float)acc;
        }
}

/* the MI355X path's arithmetic on the CPU: MXFP8(x) . decoded weights, f64 sums */
static void mxfp8_product(const float *x, int64_t m, int64_t k, const float *w, int64_t n, uint8_t *xv,
                          uint8_t *xs, float *xq, float *out)
{
    orc_quantize_mxfp8_f32(x, m, k, k, xv, xs);
    orc_mxfp8_decode(xv, xs, m, k, xq);
    dot_f64(xq, m, k, w, n, out);
}

int main(int argc, char **argv)
{
    const char *op = NULL, *model = NULL, *weight = NULL;
    uint64_t m = 0, dequant_rows = 0, iters = 20;
    int have_m = 0, have_rows = 0, have_iters = 0, benchmark = 0;
    if (argc == 2 && strcmp(argv[1], "--help") == 0) {
        fprintf(stderr,
                "Usage: %s --op matmul --model PATH --weight TENSOR_NAME --m M [--dequant-rows N] [--benchmark] "
                "[--benchmark-iters N]\n"
                "Reads exactly M*K little-endian float32 values from stdin.\n"
                "Normally writes four NumPy .npy arrays to stdout; --benchmark writes timing to stderr only.\n",
                argv[0]);
        return 0;
    }
    for (int i = 1; i < argc; ++i) {
        const char *flag = argv[i];
#define VALUE() (i + 1 < argc ? argv[++i] : (die("missing value for %s", flag), (char *)NULL))
        if (strcmp(flag, "--op") == 0) {
            if (op) die("--op specified more than once");
            op = VALUE();
        } else if (strcmp(flag, "--model") == 0) {
            if (model) die("--model specified more than once");
            model = VALUE();
        } else if (strcmp(flag, "--weight") == 0) {
            if (weight) die("--weight specified more than once");
            weight = VALUE();
        } else if (strcmp(flag, "--m") == 0) {
            if (have_m) die("--m specified more than once");
            m = parse_count(VALUE(), "M", 0);
            have_m = 1;
        } else if (strcmp(flag, "--dequant-rows") == 0) {
            if (have_rows) die("--dequant-rows specified more than once");
            dequant_rows = parse_count(VALUE(), "dequant-rows", 1);
            have_rows = 1;
        } else if (strcmp(flag, "--benchmark") == 0) {
            if (benchmark) die("--benchmark specified more than once");
            benchmark = 1;
        } else if (strcmp(flag, "--benchmark-iters") == 0) {
            if (have_iters) die("--benchmark-iters specified more than once");
            iters = parse_count(VALUE(), "benchmark-iters", 0);
            have_iters = 1;
        } else {
            die("unknown argument: %s", flag);
        }
#undef VALUE
    }
    if (!op || !model || !weight || !have_m)
        die("missing required argument; usage: %s --op matmul --model PATH --weight TENSOR_NAME --m M "
            "[--dequant-rows N] [--benchmark] [--benchmark-iters N]", argv[0]);
    if (strcmp(op, "matmul") != 0)
        die("unsupported op: %s (supported op: matmul)", op);
    if (have_iters && !benchmark)
        die("--benchmark-iters requires --benchmark");
    if (m > (1u << 24) || iters > INT_MAX)
        die("M or benchmark-iters exceed supported integer range");

    const TensorInfo t = find_tensor(model, weight);
    const int64_t k = t.k, n = t.n, mm = (int64_t)m, nb = k / IQ3S_BLOCK_VALUES;
    if (!have_rows)
        dequant_rows = (uint64_t)(n < 4 ? n : 4);
    if (dequant_rows > (uint64_t)n)
        die("dequant-rows cannot exceed tensor output width");

    uint8_t *raw = (uint8_t *)malloc(t.bytes);
    FILE *f = fopen(model, "rb");
    if (!f || fseek(f, (long)t.offset, SEEK_SET) != 0 || fread(raw, 1, t.bytes, f) != t.bytes)
        die("truncated GGUF tensor data: expected %llu bytes", (unsigned long long)t.bytes);
    fclose(f);

    const size_t in_values = (size_t)mm * (size_t)k;
    float *x = (float *)malloc(sizeof(float) * in_values);
    size_t got = fread(x, sizeof(float), in_values, stdin);
    if (got != in_values)
        die("stdin input size mismatch: expected exactly %zu bytes of row-major [M,K] float32 little-endian "
            "input, received fewer bytes", in_values * sizeof(float));
    if (fgetc(stdin) != EOF)
        die("stdin input size mismatch: expected exactly %zu bytes, received trailing bytes",
            in_values * sizeof(float));
    for (size_t i = 0; i < in_values; ++i)
        if (!isfinite(x[i]))
            die("stdin input contains a NaN or infinity");

    float *w = (float *)malloc(sizeof(float) * (size_t)(n * k));
    orc_dequant_iq3s(raw, n, nb, w);
    uint8_t *xv = (uint8_t *)malloc(in_values), *xs = (uint8_t *)malloc(in_values / 32);
    float *xq = (float *)malloc(sizeof(float) * in_values);
    float *y_mx = (float *)malloc(sizeof(float) * (size_t)(mm * n));

    if (benchmark) {
        const int warmup = 5;
        for (int i = 0; i < warmup; ++i)
            mxfp8_product(x, mm, k, w, n, xv, xs, xq, y_mx);
        double each = 0.0;
        for (uint64_t i = 0; i < iters; ++i) {
            double t0 = now_us(CLOCK_MONOTONIC);
            mxfp8_product(x, mm, k, w, n, xv, xs, xq, y_mx);
            each += now_us(CLOCK_MONOTONIC) - t0;
        }
        int threads = 1;
#ifdef _OPENMP
        threads = omp_get_max_threads();
#endif
        double c0 = now_us(CLOCK_PROCESS_CPUTIME_ID), t0 = now_us(CLOCK_MONOTONIC);
        for (uint64_t i = 0; i < iters; ++i)
            mxfp8_product(x, mm, k, w, n, xv, xs, xq, y_mx);
        double batched = (now_us(CLOCK_MONOTONIC) - t0) / (double)iters;
        double cpu = (now_us(CLOCK_PROCESS_CPUTIME_ID) - c0) / (double)iters / threads;
        fprintf(stderr,
                "benchmark backend=cpu op=matmul m=%lld n=%lld k=%lld warmup=%d iterations=%llu mean_us=%g "
                "batched_us=%g event_us=%g\n",
                (long long)mm, (long long)n, (long long)k, warmup, (unsigned long long)iters, each / (double)iters,
                batched, cpu);
        return 0;
    }
    mxfp8_product(x, mm, k, w, n, xv, xs, xq, y_mx);
    float *y_f64 = (float *)malloc(sizeof(float) * (size_t)(mm * n));
    dot_f64(x, mm, k, w, n, y_f64);

    char header[2048];
    int len = snprintf(header, sizeof header,
                       "{\"schema_version\":1,\"op\":\"matmul\",\"tensor_name\":\"%s\",\"ggml_type\":\"iq3_s\","
                       "\"shape_ggml_ne_order\":[%lld,%lld],\"row_bytes\":%llu,\"tensor_bytes\":%llu,"
                       "\"data_offset_absolute\":%llu,\"backend\":\"cpu\",\"arrays\":["
                       "{\"name\":\"dequant_rows\",\"dtype\":\"float32\",\"shape\":[%llu,%lld],\"nbytes\":%llu},"
                       "{\"name\":\"ggml_dequant_f64\",\"dtype\":\"float32\",\"shape\":[%lld,%lld],\"nbytes\":%llu},"
                       "{\"name\":\"mxfp8_f64\",\"dtype\":\"float32\",\"shape\":[%lld,%lld],\"nbytes\":%llu}]}",
                       weight, (long long)k, (long long)n, (unsigned long long)t.row_bytes,
                       (unsigned long long)t.bytes, (unsigned long long)t.offset, (unsigned long long)dequant_rows,
                       (long long)k, (unsigned long long)(dequant_rows * (uint64_t)k * 4), (long long)mm,
                       (long long)n, (unsigned long long)(mm * n * 4), (long long)mm, (long long)n,
                       (unsigned long long)(mm * n * 4));
    if (len <= 0 || len >= (int)sizeof header || strpbrk(weight, "\"\\") != NULL)
        die("tensor name cannot be written into the metadata");
    char shape[32];
    snprintf(shape, sizeof shape, "(%d,)", len);
    npy_header("|u1", shape);
    write_all(header, (size_t)len, "JSON metadata array");
    npy_f32(w, (int64_t)dequant_rows, k);
    npy_f32(y_f64, mm, n);
    npy_f32(y_mx, mm, n);
    if (fflush(stdout) != 0)
        die("failed while flushing NumPy arrays to stdout");
    return 0;
}
