/*
 * libmambo_hip: C ABI of the MI355X (gfx950) fused IQ3_S x MXFP8 projection path.
 *
 * Conventions
 *   - Every pointer argument named as a tensor is a device pointer owned by the
 *     caller; the library never allocates or frees caller memory and never
 *     synchronises the host. Work is ordered on `stream` (NULL = default stream).
 *   - Strides (ld*) count elements of the pointed-to type.
 *   - Return value: MAMBO_OK (0) or a negative MAMBO_ERR_* class; the message is
 *     available from mambo_last_error() on the calling thread. No C++ exception
 *     crosses this boundary. The Python layer maps ERR_VALUE -> ValueError,
 *     ERR_TYPE -> TypeError, everything else -> RuntimeError, as the reference
 *     launchers raise them.
 *   - A call that launches kernels first takes the thread's pending HIP error
 *     (hipGetLastError), so the failures it reports are its own; an error left pending
 *     by earlier, unrelated HIP work is then gone from hipGetLastError, and the call,
 *     if it succeeds, names it in mambo_last_error().
 *
 * Each entry point names the reference interface it replaces (paths are in the
 * Menooker/Mambo reference). The reference launches cuTile kernels with
 * ct.launch(stream, grid, kernel, args); its AOT ABI (cutile_to_cubin.py:83-95)
 * expands every array into (ptr, shape..., stride...). This ABI passes the same
 * data as plain pointers, sizes and row strides.
 */
#ifndef MAMBO_HIP_H
#define MAMBO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *mambo_stream_t; /* == hipStream_t */

enum {
    MAMBO_OK = 0,
    MAMBO_ERR_VALUE = -1,       /* bad shape, dtype, stride, alignment or config */
    MAMBO_ERR_TYPE = -2,        /* wrong kind of argument (e.g. unprepared weight) */
    MAMBO_ERR_RUNTIME = -3,     /* HIP runtime / launch failure */
    MAMBO_ERR_UNSUPPORTED = -4  /* device is not gfx950 */
};

enum {
    MAMBO_DTYPE_F32 = 0,
    MAMBO_DTYPE_BF16 = 1,
    MAMBO_DTYPE_MXFP8 = 2 /* E4M3 values plus E8M0 scales per 32 (mambo_chain_launch only) */
};

/* Kernel families of the projection. */
enum {
    MAMBO_GEMM_AUTO = 0,    /* library default for the shape */
    MAMBO_GEMM_STREAM = 1,  /* weight-streaming kernel, block-diagonal activations (M <= 4 per MFMA) */
    MAMBO_GEMM_TILED = 2,   /* LDS-tiled kernel for large M */
    MAMBO_GEMM_DENSE = 3    /* weight-streaming kernel, dense 16-token activations, exact two-term weights */
};

/* Tunable launch configuration of mambo_iq3s_fp8_matmul (the autotuner's search
 * space; replaces the cuTile tile_m/tile_n/split_k/occupancy hints of
 * iq3_s_fp8.py:49-58,402-465). Zero fields (and kernel == MAMBO_GEMM_AUTO) take the
 * value of mambo_gemm_default_config for the shape. */
typedef struct mambo_gemm_config {
    int32_t kernel;  /* MAMBO_GEMM_* */
    int32_t waves;   /* waves (64 lanes) per workgroup */
    int32_t split_k; /* workgroups sharing one output tile along K (f32 atomics) */
    int32_t tile_m;  /* TILED: rows of M per workgroup */
    int32_t tile_n;  /* TILED: rows of N per workgroup (16/32-token tiles: per K group of waves;
                        waves beyond one group split the workgroup's K blocks) */
    int32_t reserved[3];
} mambo_gemm_config;

/* Last error message of the calling thread ("" if none). */
const char *mambo_last_error(void);

/* ABI version (major * 100 + minor). */
int mambo_abi_version(void);

/* Architecture the device code was built for ("gfx950"). */
const char *mambo_build_arch(void);

/* Writes the gcnArchName of `device` (e.g. "gfx950:sramecc+:xnack-") into buf. */
int mambo_device_arch(int device, char *buf, int buf_len);

/* Host copies of the codebook: iq3s_grid (iq3_s_fp8.py:63-74, `iq3_s_table`) and its
 * E4M3-encoded form (iq3_s_fp8.py:77-94, `iq3_s_fp8_table`). out: uint32[512]. */
int mambo_iq3s_grid(uint32_t *out);
int mambo_iq3s_fp8_grid(uint32_t *out);

/* The exact two-term split of IQ3_S weight magnitudes used by the dense kernels (no
 * reference counterpart; exported so it can be checked without a GPU). out: uint32[64];
 * out[4*s + 0..1] hold the E4M3 bytes of hi/2 for grid levels 0..7 (byte j of word w is
 * level 4w + j) and out[4*s + 2..3] those of lo/2, where (1 + 2s)(2l + 1) = hi + lo and
 * hi is rounded to 4 significant bits (ties to even). */
int mambo_iq3s_split_table(uint32_t *out);

/* MXFP8 activation quantizer. Replaces launch_quantize_fp8 / quantize_activation_fp8
 * (quantize_fp8.py:42-52,67-84). x: [m, ldx] of f32 or bf16 (x_dtype); per 32
 * consecutive K elements writes one E8M0 scale byte (scales[m, lds]) and 32 E4M3
 * bytes (values[m, ldv]): e = max(ceil(log2(amax/448)), -127) computed exactly
 * (0 for an all-zero block), q = E4M3(x * 2^-e) with round-to-nearest-even.
 * k % 32 == 0; m >= 1. */
int mambo_quantize_mxfp8(const void *x, int x_dtype, int64_t m, int64_t k, int64_t ldx,
                         uint8_t *values, int64_t ldv, uint8_t *scales, int64_t lds,
                         mambo_stream_t stream);

/* Bytes of the private tile layout for an [n, blocks] IQ3_S weight. */
int64_t mambo_iq3s_packed_bytes(int64_t n, int64_t blocks);

/* Split raw GGUF IQ3_S blocks into the reference's SoA fields and/or the private tile
 * layout. Replaces prepare_iq3_s_fields (iq3_s_weight.py:25-54). raw byte (r, b, i) is
 * at raw + r*stride_n + b*stride_b + i*stride_byte (any alignment). Outputs (each may
 * be NULL, but not all): d u16[blocks, n], qs u32[blocks, n, 16], qh u16[blocks, n, 4],
 * signs i32[blocks, n, 8], scales u32[blocks, n] (IQ3SFields, iq3_s_weight.py:10-23),
 * packed u8[mambo_iq3s_packed_bytes(n, blocks)]. */
int mambo_iq3s_prepare(const uint8_t *raw, int64_t n, int64_t blocks, int64_t stride_n,
                       int64_t stride_b, int64_t stride_byte, uint16_t *d, uint32_t *qs,
                       uint16_t *qh, int32_t *signs, uint32_t *scales, uint8_t *packed,
                       mambo_stream_t stream);

/* Build the tile layout from SoA fields (for IQ3SFields built by other means). */
int mambo_iq3s_pack(const uint16_t *d, const uint32_t *qs, const uint16_t *qh,
                    const int32_t *signs, const uint32_t *scales, int64_t n, int64_t blocks,
                    uint8_t *packed, mambo_stream_t stream);

/* Standalone decoder. Replaces launch_dequant_iq3_s / decode_iq3_s_blocks
 * (iq3_s_fp8.py:202-222,341-351): values u8[n, blocks*256] = E4M3 bits of
 * sign * grid magnitude, out_scales f32[n, blocks*8] = f32(d) * (1 + 2*s). */
int mambo_iq3s_dequant(const uint16_t *d, const uint32_t *qs, const uint16_t *qh,
                       const int32_t *signs, const uint32_t *scales, int64_t n, int64_t blocks,
                       uint8_t *values, float *out_scales, mambo_stream_t stream);

/* Fused projection out[m, n] (f32, row stride ldo) = sum over K of
 * MXFP8(x)[m, k] * IQ3_S(w)[n, k]. Replaces launch_iq3_s_fp8_matmul with
 * iq3_s_fp8_matmul / iq3_s_fp8_matmul_medium (iq3_s_fp8.py:225-333,364-399).
 * xv u8[m, ldxv] E4M3, xs u8[m, ldxs] E8M0 (K = blocks*256, K/32 scales per row);
 * packed: tile layout from mambo_iq3s_prepare/mambo_iq3s_pack.
 * xv and ldxv must be 16-byte aligned; configurations of the tiled kernel
 * (MAMBO_GEMM_TILED, which the default picks from 17 tokens on) also need xs and ldxs
 * 8-byte aligned and return MAMBO_ERR_VALUE otherwise (the stream and dense kernels take
 * any xs). cfg may be NULL (library default). When the
 * chosen configuration splits K, `out` is zeroed on `stream` first and partial sums are
 * added with f32 atomics (results then vary in the last bits from run to run, as the
 * reference's split-K does). */
int mambo_iq3s_fp8_matmul(const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs,
                          int64_t m, const uint8_t *packed, int64_t n, int64_t blocks,
                          float *out, int64_t ldo, const mambo_gemm_config *cfg,
                          mambo_stream_t stream);

/* Up to MAMBO_MAX_GROUP projections of the same activations in one launch. No
 * reference counterpart: the reference calls launch_iq3_s_fp8_matmul once per weight
 * (iq3_s_fp8.py:364-399). This is for callers whose projections share an input, such
 * as q/k/v of an attention block or gate/up of an MLP: the result equals one
 * mambo_iq3s_fp8_matmul per projection, with one launch ramp instead of `count`. */
#define MAMBO_MAX_GROUP 4
typedef struct mambo_projection {
    const uint8_t *packed; /* packed weight, n rows x blocks */
    int64_t n;             /* output features of this projection */
    float *out;            /* f32 [m, ldo] */
    int64_t ldo;           /* >= n */
} mambo_projection;

/* proj[0..count) share xv/xs and K = blocks*256; cfg as for mambo_iq3s_fp8_matmul, with
 * the default computed for the summed N (mambo_gemm_default_config(m, sum of n, ...)). */
int mambo_iq3s_fp8_matmul_grouped(const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs,
                                  int64_t m, const mambo_projection *proj, int count, int64_t blocks,
                                  const mambo_gemm_config *cfg, mambo_stream_t stream);

/* Quantize + matmul in one call (no reference counterpart: the reference quantizes in a
 * launch of its own, quantize_fp8.py:1-4, then calls iq3_s_fp8_matmul; this is the
 * fused activation-quantize prologue for decode M). x: unquantized activations [m, K]
 * (MAMBO_DTYPE_F32 or _BF16, row stride ldx elements); proj/count/blocks/cfg as for
 * mambo_iq3s_fp8_matmul_grouped. For M <= 4 on the stream kernel with its rows staged in
 * LDS (and x 16-byte aligned) every workgroup quantizes the rows into its LDS copy with
 * the quantizer's arithmetic - one launch, results bit-identical to the two-step path
 * with the same cfg - and xv/xs are not touched; otherwise mambo_quantize_mxfp8 writes
 * the caller's MXFP8 buffers xv [m, ldxv] / xs [m, ldxs] and the GEMM reads them. */
int mambo_iq3s_matmul_quantize_grouped(const void *x, int x_dtype, int64_t ldx, int64_t m,
                                       const mambo_projection *proj, int count, int64_t blocks,
                                       const mambo_gemm_config *cfg, uint8_t *xv, int64_t ldxv,
                                       uint8_t *xs, int64_t ldxs, mambo_stream_t stream);

/* Chained projections for 1..4 tokens: up to MAMBO_MAX_CHAIN launches, each as
 * mambo_iq3s_fp8_matmul_grouped (1..MAMBO_MAX_GROUP projections of one input), run in
 * order in ONE launch of the block-diagonal streaming kernel. No reference counterpart:
 * the reference runs one launch_iq3_s_fp8_matmul per weight (iq3_s_fp8.py:364-399); this
 * is for callers that run many projections back to back at decode sizes, such as a
 * layer's q/k/v, o, gate/up and down or several layers. The outputs equal those of the
 * separate grouped launches on one stream with the stream kernel at cfg->waves (4, 8 or
 * 16) and no K split, bit for bit. Order: launch i reads its activations only after every
 * output of launches < i is stored (device counters in `sync`), so launch i may take as
 * its activations f32 or bf16 outputs of an earlier launch (x_dtype F32/BF16: rows
 * quantized to MXFP8 in the kernel with the quantizer's arithmetic) - the semantics of
 * the same launches on one stream. The workgroups of launch i+1 start streaming their
 * weights while launch i drains. Every dependency wait is bounded (cfg->timeout_us,
 * default 2 s); a wait that times out is reported by mambo_chain_status, the outputs then
 * being undefined.
 * sync: MAMBO_CHAIN_SYNC_WORDS uint32 of device memory (16.5 KiB: counters spread over
 * lines of their own), zero before the first call; every call that does not time out
 * leaves them zero again (a timeout is kept until mambo_chain_status reads it, which then
 * clears every word). Calls that overlap in time must use different sync words.
 * Allocates nothing. Measured slower than the same launches one by one on the Llama-3
 * sweeps at 1 token (70B 0.92x, 8B 0.86x): it is the ordered-dependency form, not the
 * fast path. */
#define MAMBO_MAX_CHAIN 16
#define MAMBO_CHAIN_SYNC_WORDS 4224
typedef struct mambo_chain_launch {
    const void *x;       /* MXFP8 values u8[m, ldx] (x_dtype MAMBO_DTYPE_MXFP8), or f32/bf16 rows */
    int32_t x_dtype;     /* MAMBO_DTYPE_MXFP8, MAMBO_DTYPE_F32 or MAMBO_DTYPE_BF16 */
    int32_t count;       /* projections in proj */
    int64_t ldx;         /* row stride of x in elements; MXFP8: 16-byte multiple, else rows 16-byte aligned */
    const uint8_t *xs;   /* MXFP8 only: E8M0 scales u8[m, ldxs], base and ldxs 4-byte aligned */
    int64_t ldxs;
    int64_t blocks;      /* K / 256 of this launch */
    mambo_projection proj[MAMBO_MAX_GROUP];
} mambo_chain_launch;
typedef struct mambo_chain_config {
    int32_t waves;               /* waves per workgroup: 4, 8 or 16 (0: 4) */
    int32_t tiles_per_workgroup; /* 16-row weight tiles each workgroup takes (0: 1) */
    int64_t timeout_us;          /* bound of each dependency wait, at most 60 s (0: 2 s) */
    int32_t wait_bias;           /* tests only: added to every wait's target, so waits time out */
    int32_t reserved[3];
} mambo_chain_config;
int mambo_iq3s_fp8_matmul_chain(int64_t m, const mambo_chain_launch *launches, int count,
                                const mambo_chain_config *cfg, uint32_t *sync, mambo_stream_t stream);

/* Reads the status of the chained calls that used `sync` (synchronously: it waits for the
 * device copy). MAMBO_ERR_RUNTIME when a dependency wait timed out (all sync words are then
 * cleared: after a timeout, launches may have finished out of order) or when the counters
 * are not zero; else MAMBO_OK. */
int mambo_chain_status(uint32_t *sync);

/* mambo_iq3s_matmul_quantize_grouped without the caller's MXFP8 buffers: allocates
 * nothing (no hipMalloc, no allocating library call). No reference counterpart; for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid it). Where the rows are not quantized inside the GEMM (M > 4,
 * unaligned rows, rows too long for LDS) their MXFP8 form is staged in a device array
 * the library holds once per GPU (MAMBO_NOALLOC_SCRATCH_BYTES, until the process ends):
 * calls needing more than that (m*K + m*K/32 bytes, K = blocks*256) return
 * MAMBO_ERR_VALUE. Every call on a GPU shares that GPU's array, so calls that overlap in
 * time on one GPU (on different streams) race; calls ordered on one stream do not. The
 * results equal mambo_iq3s_matmul_quantize_grouped's with the same cfg. */
#define MAMBO_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int mambo_iq3s_matmul_quantize_grouped_noalloc(const void *x, int x_dtype, int64_t ldx, int64_t m,
                                               const mambo_projection *proj, int count, int64_t blocks,
                                               const mambo_gemm_config *cfg, mambo_stream_t stream);

/* The configuration mambo_iq3s_fp8_matmul uses when cfg == NULL. */
int mambo_gemm_default_config(int64_t m, int64_t n, int64_t blocks, mambo_gemm_config *out);

/* Validates cfg for the shape (MAMBO_OK or MAMBO_ERR_VALUE with a reason). */
int mambo_gemm_check_config(int64_t m, int64_t n, int64_t blocks, const mambo_gemm_config *cfg);

/* Autotuner candidates for the shape (replaces the search-space construction of
 * make_benchmark_cases, iq3_s_fp8.py:402-465): writes the first min(count, capacity)
 * configurations to out (out may be NULL when capacity is 0) and returns count, or a
 * negative status. out[0] is the library default (all fields 0, MAMBO_GEMM_AUTO); every
 * other entry passes mambo_gemm_check_config for (m, n, blocks). */
int64_t mambo_gemm_config_enumerate(int64_t m, int64_t n, int64_t blocks, mambo_gemm_config *out,
                                    int64_t capacity);

/* Synthetic inputs for benchmarks and full-size checks (no reference counterpart; the
 * reference draws them with numpy/cupy RNGs, test_iq3_s_fp8.py:41-51). Counter-based:
 *   rnd(seed, stream, i) = splitmix64(splitmix64(seed*0xD1B54A32D192ED03 + stream) + i);
 *   normal(seed, stream, i) = (sum_{t<12} (rnd(seed, stream, 12i+t) >> 32) - 6*2^32) / 2^32.
 * mambo_synth_iq3s: raw u8[nrows, blocks, 110] for weight rows [row0, row0+nrows):
 *   bytes 2..109 of block (r, b) = bytes of rnd(seed, 1, 14*(r*blocks+b) + j/8);
 *   d = fp16(f32(|normal(seed, 2, r*blocks+b)| * 2e-3)).
 * mambo_synth_bf16: out[i] = bf16(f32(normal(seed, 3, i0+i) * (outlier ? 100 : 1))),
 *   outlier iff (rnd(outlier_seed, 4, i0+i) >> 11) < outlier_frac * 2^53. */
int mambo_synth_iq3s(uint64_t seed, int64_t blocks, int64_t row0, int64_t nrows, uint8_t *raw,
                     mambo_stream_t stream);
int mambo_synth_bf16(uint64_t seed, uint64_t outlier_seed, double outlier_frac, int64_t i0,
                     int64_t count, uint16_t *out, mambo_stream_t stream);

/* Diagnostic: element-wise f32 -> E4M3 through the kernels' integer rounding path
 * (out_sw) and the hardware v_cvt_pk_fp8_f32 (out_hw); either output may be NULL.
 * Used to check the hardware conversion against the integer restatement. */
int mambo_e4m3_convert(const float *in, int64_t n, uint8_t *out_sw, uint8_t *out_hw,
                       mambo_stream_t stream);

/* Fill n floats with `value` (a kernel, not hipMemsetAsync, so it may be captured in
 * a HIP graph). */
int mambo_fill_f32(float *ptr, int64_t n, float value, mambo_stream_t stream);

/* Diagnostic: copy `bytes` (a multiple of 16, both pointers 16-byte aligned) from src to
 * dst with 16-byte vector loads and stores, each byte read and written exactly once. A
 * plain stream of known size, used to calibrate the HBM byte counters (FETCH_SIZE,
 * WRITE_SIZE) that the kernels' traffic figures are scaled by. */
int mambo_copy_bytes(const void *src, void *dst, int64_t bytes, mambo_stream_t stream);

/* Diagnostic: read `bytes` (a multiple of 16, src 16-byte aligned) with 16-byte vector
 * loads over a grid of MAMBO_READ_SINK_WORDS threads; thread t writes the XOR of the
 * 32-bit words of the chunks t, t + MAMBO_READ_SINK_WORDS, ... to sink[t], so `sink`
 * holds MAMBO_READ_SINK_WORDS uint32 and the XOR of all of them is the XOR of the input.
 * The plain-read ceiling that the weight streams are compared with. */
#define MAMBO_READ_SINK_WORDS (2048 * 256)
int mambo_read_bytes(const void *src, int64_t bytes, uint32_t *sink, mambo_stream_t stream);

/* Diagnostic: scaled-MFMA throughput on this device. `workgroups` x 4 waves each run
 * `iters` rounds of eight independent v_mfma_scale_f32_16x16x128_f8f6f4 chains (2*16*16*128
 * flops per MFMA); out must hold workgroups * 256 floats and receives 4096 * iters in
 * every element. */
int mambo_mfma_peak(int64_t workgroups, int iters, float *out, mambo_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBO_HIP_H */
