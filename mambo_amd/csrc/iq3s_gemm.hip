// Fused IQ3_S x MXFP8 projection for gfx950: out[m, n] = sum_k x[m, k] * w[n, k].
//
// Reference semantics (src/python/mambo/kernels/iq3_s_fp8.py:225-333): per 32-weight
// group, an FP8 block-scaled MMA of the E4M3 activation codes (E8M0 scale per
// activation group) with the E4M3 grid magnitudes (weight scale 1.0), then the f32
// post-scale F = d * (1 + 2*nibble) of the weight group, accumulated over groups.
//
// Streaming kernel (this file, all M; one pass over the weights per 16 rows of M).
// One wave owns a 16-row weight tile and walks super-blocks along K; the workgroup's
// waves split the blocks of one K range and reduce through LDS; several workgroups may
// split K further (f32 atomics into a zeroed output).
//
// Per super-block each lane decodes 16 four-weight codes of row col (q = lane/16, col =
// lane%16) straight into the B operand of V_MFMA_SCALE_F32_16X16X128_F8F6F4: lane l of
// B holds 32 bytes of column col (K [16q, 16q+16) and [64+16q, 64+16q+16), byte t of
// lane l of A pairing with byte t of lane l' of B for l >> 4 == l' >> 4), and the tile
// layout (mambo_common.h) stores each lane's codes in exactly that order, so the decoded
// words are its B slice as they are; nothing decoded touches HBM. Layout measured on
// gfx950 with one-hot operands.
//   code address: 2 VALU (funnel shift + mask of the 9-bit index stream)
//   magnitude:    1 LDS read of the E4M3-encoded grid word
//   signs:        2 VALU (rotate the bit-transposed sign word, bit-field insert)
// Because F differs per 32-weight group and a K=128 MFMA spans four groups (one per K
// block of 32), the A operand (activations) is block-diagonal: row i = 4*g + m' of A
// holds activation row m' only in one K block (zero elsewhere), the block whose groups
// make up scale byte g (out_block). Output row (g, m'), held by lane group g, then sums
// exactly one group of its column, and each lane post-scales its own accumulator by the
// F of the scale byte it loaded itself; the four K blocks' partials are summed at the end.
// M up to 4 per MFMA, up to 16 per pass (U = 1..4 MFMAs per K step).
#include <mutex>

#include "iq3s_stream.h"

namespace {

// Workgroup (x, y, z) computes tiles [x*tpw, x*tpw + tpw) of the launch over K blocks
// [y*bps, y*bps + bps) for tokens [16z, 16z + 4U). Its W waves split each tile's blocks
// (wave w takes blocks w, w + W, ...) and stream the tiles back to back through one
// register ring, so the ring does not drain between tiles and the activations are
// staged in LDS once per workgroup. kQ != 0: xv holds unquantized rows (kQ = 1 bf16,
// 2 f32; ldxv in elements) that the workgroup quantizes to MXFP8 into its LDS copy
// itself (quantize_group32: the quantizer's arithmetic, so the codes are identical), in
// place of a separate quantizer launch; xs is unused.
// kLg: log2 of the codebook copies in LDS (see RepGrid).
// At most 256 registers per lane (two waves per SIMD): the compiler then keeps the MFMA
// results in VGPRs. Allowed the full 512 of one wave per SIMD (4-wave workgroups), it
// wrote them to AGPRs and read each back (8 v_accvgpr_read per block) and needed 84
// registers instead of 71 at one token: 70B M=1 sweep +0.5%, M=2 +1.2%, 8B M=1 +0.7%.
template <int U, int W, bool kLdsAct, int kQ = 0, int kLg = 0>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2))) void gemm_stream_kernel(const uint8_t *__restrict__ xv, int64_t ldxv,
                                                             const uint8_t *__restrict__ xs, int64_t ldxs, int64_t M,
                                                             GroupArgs ga, int64_t ntiles, int tpw, int B, int bps,
                                                             int atomic)
{
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); // wave-uniform: scalar loop control
    const int K = B * 256;
    const int64_t m0 = (int64_t)blockIdx.z * 16;
    const int rows = (int)min<int64_t>(U * 4, M - m0);
    const StreamLds L = stream_lds(U, W, rows, K, kLdsAct);
    const int64_t t_begin = (int64_t)blockIdx.x * tpw;
    const int ntw = (int)min<int64_t>(tpw, ntiles - t_begin);
    const int b_begin = blockIdx.y * bps;
    const int b_end = min(B, b_begin + bps);
    // steps per tile, the same for every wave (blocks past b_end count with a zero scale)
    const int steps = (b_end - b_begin + W - 1) / W;
    const int total = ntw * steps;
    const int first = b_begin + wave;
    const int col = lane & 15, q = lane >> 4;

    // Staging copies (codebook, activation rows and their scales) go from global memory
    // straight into LDS ahead of the ring's first weight loads: vector memory counts
    // complete in issue order, so the barrier below waits for the copies (L2) and not for
    // the weights (HBM), which stay in flight across it.
    __shared__ __align__(16) uint32_t s_grid[512 << kLg];
    const uint8_t *lut = reinterpret_cast<const uint8_t *>(s_grid);
    const uint32_t c4 = 4u * (uint32_t)(lane & ((1 << kLg) - 1));
    static_assert(kQ == 0 || kLdsAct, "quantizing rows needs the LDS copy");
    const int qgroups = rows * (K / 32); // kQ: 32-element groups to quantize
    float qv[32];
    {
        const __amdgpu_buffer_rsrc_t gr = byte_rsrc(rep_grid<kLg>());
        if constexpr (kLg == 0) { // one copy: 4-byte copies spread over up to 8 waves
            for (int i = wave; i < 8; i += W)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (lds_ptr)(s_grid + 64 * i), 4, 4u * lane, 256u * i, 0, 0);
        } else {
            for (int i = wave; i < stream_lut_bytes(kLg) / 1024; i += W)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (lds_ptr)(s_grid + 256 * i), 16, 16u * lane, 1024u * i, 0,
                                                         0);
        }
        if constexpr (kQ != 0) {
            // the first group this thread quantizes: its loads go out before the ring's
            // weight loads, so waiting for them leaves the weights in flight
            if (tid < qgroups)
                load_group32<kQ == 1>(xv, (m0 + tid / (K / 32)) * ldxv + 32 * (tid % (K / 32)), qv);
        }
        if constexpr (kLdsAct && kQ == 0) {
            // activation rows m0 .. m0+rows-1 as 16-byte chunks (K is a multiple of 256, so
            // none straddles rows; slot c of row r takes chunk act_slot(c, r)), then their
            // scales as dwords (K/32 is a multiple of 8; the host stages only 4-byte aligned
            // scale rows)
            const int nx = rows * K / 16;
            const __amdgpu_buffer_rsrc_t xr = byte_rsrc(xv + m0 * ldxv);
            for (int i = wave; 64 * i < nx; i += W) {
                const int c = 64 * i + lane, r = c * 16 / K;
                if (c < nx)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        xr, (lds_ptr)(smem + L.x + 1024 * i), 16,
                        (uint32_t)(r * ldxv + 16 * act_slot(c - r * (K / 16), r)), 0, 0, 0);
            }
            const int ns = rows * (K / 128);
            const __amdgpu_buffer_rsrc_t sr = byte_rsrc(xs + m0 * ldxs);
            for (int i = wave; 64 * i < ns; i += W) {
                const int e = 64 * i + lane, r = e / (K / 128);
                if (e < ns)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(smem + L.xs + 256 * i), 4,
                                                             (uint32_t)(r * ldxs + 4 * (e - r * (K / 128))), 0, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // Ring of kDepth register sets with fixed slots (the loop body is unrolled kDepth
    // times): step s is decoded while steps s+1 .. s+kDepth-1 are in flight.
    WTile wr[kDepth];
    StreamCursor pc = {0, 0, t_begin, byte_rsrc(tile_ref(ga, t_begin, B).w)};
#pragma unroll
    for (int j = 0; j < kDepth - 1; ++j) {
        wr[j] = load_w_rsrc(pc.w, (uint32_t)min(first + pc.i * W, b_end - 1) * kTileBytes, lane, col);
        advance(pc, total, steps, ga, B);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (tid < 20)
        reinterpret_cast<uint32_t *>(smem + L.zero)[tid] = tid < 16 ? 0u : 0x7F7F7F7Fu;
    if constexpr (kQ != 0) {
        // rows [m0, m0+rows) to E4M3 + E8M0 in the layout the staging copies produce
        for (int gi = tid; gi < qgroups; gi += W * 64) {
            const int r = gi / (K / 32), g = gi - r * (K / 32);
            if (gi != tid)
                load_group32<kQ == 1>(xv, (m0 + r) * ldxv + 32 * g, qv);
            uint32_t codes[8];
            const int scale = quantize_group32(qv, codes);
            uint4 *dst = reinterpret_cast<uint4 *>(smem + L.x + r * K + 16 * act_slot(2 * g, r));
            dst[0] = uint4{codes[0], codes[1], codes[2], codes[3]};
            dst[1] = uint4{codes[4], codes[5], codes[6], codes[7]};
            smem[L.xs + r * (K / 32) + g] = (uint8_t)scale;
        }
    }
    // this wave's copies are done once at most the ring's kWLoads * (kDepth - 1) weight
    // loads are outstanding (s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt 6:4 and
    // lgkmcnt 11:8 left unconstrained)
    static_assert(kWLoads * (kDepth - 1) < 16, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((kWLoads * (kDepth - 1)) | (7 << 4) | (15 << 8));
    __syncthreads();

    const uint8_t *azero;
    if constexpr (kLdsAct)
        azero = smem + L.zero;
    else
        azero = g_zero_chunk;
    ALane al[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = 4 * u + (lane & 3); // row within the chunk
        if constexpr (kLdsAct)
            al[u] = a_lane<true>(lane, r < rows, smem + L.x + r * K, smem + L.xs + r * (K / 32), smem + L.zero,
                                 smem + L.zero + 64);
        else
            al[u] = a_lane<false>(lane, r < rows, xv + (m0 + r) * ldxv, xs + (m0 + r) * ldxs, g_zero_chunk,
                                  g_unit_scales);
    }

    float acc[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[u][r] = 0.0f;

    // Activations staged in LDS are read at decode time; otherwise they ride in the ring
    // with the weights (the first kDepth-1 of them are read here, after the staging).
    ATile<U> ar[kLdsAct ? 1 : kDepth];
    if constexpr (!kLdsAct) {
        int as = 0, ai = 0; // the prefetch cursor's (s, i) for these first steps
#pragma unroll
        for (int j = 0; j < kDepth - 1; ++j) {
            load_a<U, kLdsAct>(ar[j], al, min(first + ai * W, b_end - 1), azero);
            if (as + 1 < total) {
                ++as;
                if (++ai == steps)
                    ai = 0;
            }
        }
    }
    float *red = reinterpret_cast<float *>(smem + L.red);
    int ci = 0, tile_no = 0; // step within the tile being decoded, and its index in the run
    for (int s0 = 0; s0 < total; s0 += kDepth) {
#pragma unroll
        for (int j = 0; j < kDepth; ++j) {
            const int s = s0 + j;
            const int slot = (j + kDepth - 1) % kDepth;
            const int bp = min(first + pc.i * W, b_end - 1);
            wr[slot] = load_w_rsrc(pc.w, (uint32_t)bp * kTileBytes, lane, col);
            if constexpr (!kLdsAct)
                load_a<U, kLdsAct>(ar[slot], al, bp, azero);
            advance(pc, total, steps, ga, B);
            // keep the prefetch issued before the decode of step s (scheduler fence)
            if constexpr (MAMBO_SCHED_FENCE)
                __builtin_amdgcn_sched_barrier(0);
            // steps past the run (the ring's tail) skip the math; the condition is uniform
            // over the workgroup, so the tile-end barrier inside is reached by every wave
            if (s < total) {
                const int blk = first + ci * W;
                if constexpr (kLdsAct) {
                    // the activation reads go out before the codebook reads: LDS reads
                    // complete in order, so the decode's partial waits then never wait
                    // for them (left to the scheduler, they sank behind the codebook
                    // reads; without this fence the one-token sweep measured 0.2% slower)
                    load_a<U, kLdsAct>(ar[0], al, min(blk, b_end - 1), azero);
                    __builtin_amdgcn_sched_barrier(0);
                    compute_block<U, kLg>(wr[j], ar[0], lut, c4, acc, blk < b_end);
                } else {
                    compute_block<U, kLg>(wr[j], ar[j], lut, c4, acc, blk < b_end);
                }
                if (++ci == steps) {
                    stream_tile_end<U, W>(acc, red + (tile_no & 1) * (W * U * 64), wave, tid, lane,
                                          tile_ref(ga, t_begin + tile_no, B), m0, M, atomic);
                    ci = 0;
                    ++tile_no;
                }
            }
            if constexpr (MAMBO_SCHED_FENCE)
                __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// ============================================================================ dense kernel
// For M > 4 the block-diagonal operand above wastes 3/4 of every MFMA and needs one A
// sub-tile per 4 tokens. The dense kernel feeds 16 real tokens as the A operand, so one
// K=128 MFMA spans four weight groups with different scales (1+2s); the weight operand
// then carries the exact per-weight product P = (1+2s)*g as two E4M3 terms
// (hi/2 + lo/2, B scale 2; see SplitTables) and the block's fp16 d is applied in f32.
// Per 256-weight block: 4 MFMAs (2 K halves x hi/lo) for 16 tokens.
//
// Decode per code: the grid word in level form (bytes 0..7) from LDS selects, with one
// v_perm_b32 each, the hi and lo bytes of four weights from the group's 16-byte split
// table entry; the four signs are OR-ed into hi and XOR-ed into lo (lo has a sign).
// The tile layout puts each lane's codes in the MFMA's K order (mambo_common.h): in MFMA
// h the K blocks hold weight groups (kb0, kb1, kb2, kb3) = (h, 4+h, 2+h, 6+h), each group
// inside one K block (one E8M0 activation scale per K block), and lane (col, q) decodes
// half q&1 of groups 4*(q>>1) + h (bytes 0-15) and 4*(q>>1) + 2 + h (bytes 16-31): the
// decoded words are its operand as they are. The A operand of lane (token i, q) takes
// the matching bytes: group 4*(q>>1) + h, half q&1, and +64 bytes for group 4*(q>>1) +
// 2 + h. Scale lane i + 16*kb holds token i's scale of group h + 4*(kb&1) + 2*(kb>>1).

struct ADense {
    v8i a[2];
    uint8_t s[2];
};

// Activation bytes and scales of one lane at block b: base + off + 256*b (values) and
// sbase + soff + 8*b (scales), with wave-uniform bases and 32-bit lane offsets.
__device__ __forceinline__ void load_a_dense(ADense &at, const uint8_t *__restrict__ xbase, uint32_t xoff,
                                             const uint8_t *__restrict__ sbase, uint32_t soff, int b)
{
    const uint8_t *xp = xbase + 256 * (int64_t)b;
    const uint8_t *sp = sbase + 8 * (int64_t)b;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 lo = *reinterpret_cast<const uint4 *>(xp + (xoff + 32u * h));
        const uint4 hi = *reinterpret_cast<const uint4 *>(xp + (xoff + 32u * h + 64u));
        at.a[h] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        at.s[h] = sp[soff + h];
    }
}

// load_a_dense from global memory through buffer resources over the chunk's activation
// rows (xr) and scales (sr).
__device__ __forceinline__ void load_a_dense_rsrc(ADense &at, __amdgpu_buffer_rsrc_t xr, uint32_t xoff,
                                                  __amdgpu_buffer_rsrc_t sr, uint32_t soff, int b)
{
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const auto lo = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + 32u * h, 256u * b, 0);
        const auto hi = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + 32u * h + 64u, 256u * b, 0);
        at.a[h] = v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        at.s[h] = __builtin_amdgcn_raw_buffer_load_b8(sr, soff + h, 8u * b, 0);
    }
}

// hi and lo words of code C of a group: level bytes select from the split table entry
// (tab.x/.y: hi of levels 0-3/4-7, tab.z/.w: lo); the four signs, moved onto bits
// 7,15,23,31 by one shift of the transposed sign word, are OR-ed into hi and XOR-ed into
// lo (one v_bitop3 each: a | (b & c) = 0xF8, a ^ (b & c) = 0x78).
template <int C>
__device__ __forceinline__ void split_word(uint32_t lv, uint32_t p, uint4 tab, int &hi, int &lo)
{
    const uint32_t r = funnel_shr(p, p, (25 + C) & 31);
    hi = (int)__builtin_amdgcn_bitop3_b32(__builtin_amdgcn_perm(tab.y, tab.x, lv), r, 0x80808080u, 0xF8);
    lo = (int)__builtin_amdgcn_bitop3_b32(__builtin_amdgcn_perm(tab.w, tab.z, lv), r, 0x80808080u, 0x78);
}

// Split-table entry of operand half X (0: bytes 0-15, 1: bytes 16-31) of MFMA H, from the
// lane's dense scale word (dense_scales: nibble 2X + H).
template <int H, int X>
__device__ __forceinline__ uint4 split_entry(const uint4 *split, uint32_t sc)
{
    return split[(sc >> (4 * (2 * X + H))) & 15u];
}

// MFMA H's hi and lo operands: codes 0-3 with the entry of half 0 (ta), 4-7 of half 1 (tb).
template <int H, int... C>
__device__ __forceinline__ void decode_split(const uint32_t (&s)[5], uint32_t p, const uint8_t *lvl, uint4 ta,
                                             uint4 tb, v8i &bhi, v8i &blo, std::integer_sequence<int, C...>)
{
    int h[8], l[8];
    (split_word<C>(*reinterpret_cast<const uint32_t *>(lvl + code_addr<8 * H + C>(s)), p, C < 4 ? ta : tb, h[C],
                   l[C]),
     ...);
    bhi = v8i{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
    blo = v8i{l[0], l[1], l[2], l[3], l[4], l[5], l[6], l[7]};
}

// Both halves of one tile-block (MFMA H = 0, 1).
__device__ __forceinline__ void decode_block(const WTile &w, const uint8_t *lvl, const uint4 *split, v8i (&bh)[2],
                                             v8i (&bl)[2])
{
    const uint32_t s[5] = {w.ia.x, w.ia.y, w.ia.z, w.ia.w, (uint32_t)w.ib};
    const uint32_t sc = dense_scales(w.sc);
    decode_split<0>(s, w.sg.x, lvl, split_entry<0, 0>(split, sc), split_entry<0, 1>(split, sc), bh[0], bl[0],
                    std::make_integer_sequence<int, 8>{});
    decode_split<1>(s, w.sg.y, lvl, split_entry<1, 0>(split, sc), split_entry<1, 1>(split, sc), bh[1], bl[1],
                    std::make_integer_sequence<int, 8>{});
}

template <int MC>
__device__ __forceinline__ void compute_dense(const WTile &w, const ADense (&at)[MC], const uint8_t *lvl,
                                              const uint4 *split, float (&acc)[MC][4], bool valid)
{
    v8i bh[2], bl[2];
    decode_block(w, lvl, split, bh, bl);
    // B scale 2^1: the split terms are stored halved. Per 16-token chunk one chain of four
    // MFMAs on the one decode (the callers interleave the chains of their NT tiles).
    const float f = valid ? half_bits_to_float((uint16_t)w.dh) : 0.0f;
#pragma unroll
    for (int u = 0; u < MC; ++u) {
        const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
        v4f c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(at[u].a[0], bh[0], zero, 0, 0, 0, (int)at[u].s[0], 0, 128);
        c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(at[u].a[0], bl[0], c, 0, 0, 0, (int)at[u].s[0], 0, 128);
        c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(at[u].a[1], bh[1], c, 0, 0, 0, (int)at[u].s[1], 0, 128);
        c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(at[u].a[1], bl[1], c, 0, 0, 0, (int)at[u].s[1], 0, 128);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[u][r] = __builtin_fmaf(c[r], f, acc[u][r]);
    }
}

// Activation fragments of all MC token chunks for block b (from the LDS copy when
// kLdsAct, else from global memory through the resources xr, sr).
template <bool kLdsAct, int MC>
__device__ __forceinline__ void load_acts_dense(ADense (&a)[MC], const uint8_t *xbase, const uint8_t *sbase,
                                                __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t sr,
                                                const uint32_t (&xoff)[MC], const uint32_t (&soff)[MC], int b)
{
#pragma unroll
    for (int u = 0; u < MC; ++u) {
        if constexpr (kLdsAct)
            load_a_dense(a[u], xbase, xoff[u], sbase, soff[u], b);
        else
            load_a_dense_rsrc(a[u], xr, xoff[u], sr, soff[u], b);
    }
}

// Dynamic LDS of the dense kernel (level grid and split tables sit in static LDS):
// cross-wave partial sums [W][NT][MC][4][64] f32 and - when kLdsAct - the workgroup's
// activation rows [rows][K] and scales [rows][K/32].
struct DenseLds {
    int red, x, xs, total;
};

__host__ __device__ inline DenseLds dense_lds(int W, int NT, int MC, int rows, int K, bool lds_act)
{
    DenseLds l;
    l.red = 0;
    l.x = l.red + (W > 1 ? W * NT * MC * 4 * 64 * 4 : 0);
    l.xs = l.x + (lds_act ? rows * K : 0);
    l.total = l.xs + (lds_act ? rows * (K / 32) : 0);
    return l;
}

// A workgroup covers NT weight tiles (16*NT rows) and MC chunks of 16 tokens; each wave
// applies one activation fragment per block and chunk to all NT tiles (activation loads
// per weight byte drop by NT) and each decoded tile-block to all MC chunks (decode work
// per token drops by MC). Grouped projections start on a workgroup boundary
// (tile_begin counts workgroups).
template <int W, int NT, bool kLdsAct, int MC>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2))) void gemm_dense_kernel(
    const uint8_t *__restrict__ xv, int64_t ldxv,
                                                            const uint8_t *__restrict__ xs, int64_t ldxs, int64_t M,
                                                            GroupArgs ga, int B, int bps, int atomic)
{
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t s_lvl[512];
    __shared__ uint4 s_split[16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = B * 256;
    const int64_t m0 = (int64_t)blockIdx.z * (16 * MC);
    const int rows = (int)min<int64_t>(16 * MC, M - m0);
    const DenseLds L = dense_lds(W, NT, MC, rows, K, kLdsAct);
    const uint8_t *packed = ga.packed[0];
    float *out = ga.out[0];
    int64_t N = ga.n[0], ldo = ga.ldo[0], wg = blockIdx.x;
#pragma unroll
    for (int g = 1; g < kMaxGroup; ++g)
        if (g < ga.count && (int64_t)blockIdx.x >= ga.tile_begin[g]) {
            packed = ga.packed[g];
            out = ga.out[g];
            N = ga.n[g];
            ldo = ga.ldo[g];
            wg = blockIdx.x - ga.tile_begin[g];
        }
    const int64_t tiles = (N + kTileRows - 1) / kTileRows;
    const int b_begin = blockIdx.y * bps;
    const int b_end = min(B, b_begin + bps);
    const int col = lane & 15, q = lane >> 4;
    __amdgpu_buffer_rsrc_t wt[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) // tiles past the weight's last are clamped; stores are masked
        wt[nt] = byte_rsrc(packed + min(wg * NT + nt, tiles - 1) * (int64_t)B * kTileBytes);
    const int first = b_begin + wave;
    const int count = first < b_end ? (b_end - first + W - 1) / W : 0;
    const int last = first + (count - 1) * W;
    const uint8_t *lvl = reinterpret_cast<const uint8_t *>(s_lvl);

    // A lane of chunk u: token 16u + col, bytes of group 4*(q>>1) + h, half q&1 (+64 bytes
    // for group 4*(q>>1) + 2 + h), scale of group 4*(q&1) + 2*(q>>1) + h. Lanes of tokens
    // past M read the last token: they only feed output rows that are never stored.
    const uint32_t xo = 32u * (4 * (q >> 1)) + 16u * (q & 1), so = 4u * (q & 1) + 2u * (q >> 1);
    const uint8_t *xbase = smem + L.x, *sbase = smem + L.xs;     // kLdsAct
    __amdgpu_buffer_rsrc_t xr = byte_rsrc(xv + m0 * ldxv), sr = byte_rsrc(xs + m0 * ldxs); // otherwise
    uint32_t xoff[MC], soff[MC];
#pragma unroll
    for (int u = 0; u < MC; ++u) {
        const int rowc = min(16 * u + col, rows - 1);
        if constexpr (kLdsAct) {
            xoff[u] = (uint32_t)(rowc * K) + xo;
            soff[u] = (uint32_t)(rowc * (K / 32)) + so;
        } else {
            xoff[u] = (uint32_t)(rowc * ldxv) + xo;
            soff[u] = (uint32_t)(rowc * ldxs) + so;
        }
    }
#define load_acts(a, b) load_acts_dense<kLdsAct, MC>(a, xbase, sbase, xr, sr, xoff, soff, b)

    // Staging copies (level grid, split table and - when kLdsAct - the activation rows
    // and scales) go from global memory straight into LDS ahead of the ring's first
    // weight loads: vector memory counts complete in issue order, so the barrier waits
    // for the copies (L2) and not for the weights (HBM), which stay in flight across it.
    {
        const __amdgpu_buffer_rsrc_t gr = byte_rsrc(c_grid.level), tr = byte_rsrc(&c_split.w[0][0]);
        for (int i = wave; i < 9; i += W) {
            if (i < 8)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (lds_ptr)(s_lvl + 64 * i), 4, 4u * lane, 256u * i, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(tr, (lds_ptr)s_split, 4, 4u * lane, 0, 0, 0);
        }
        if constexpr (kLdsAct) {
            // rows as 16-byte chunks (K is a multiple of 256, so none straddles rows), then
            // their scales as dwords (K/32 is a multiple of 8; the host stages only 4-byte
            // aligned scale rows)
            const int nx = rows * K / 16;
            for (int i = wave; 64 * i < nx; i += W) {
                const int c = 64 * i + lane, r = c * 16 / K;
                if (c < nx)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(smem + L.x + 1024 * i), 16,
                                                             (uint32_t)(r * ldxv + (c * 16 - r * K)), 0, 0, 0);
            }
            const int ns = rows * (K / 128);
            for (int i = wave; 64 * i < ns; i += W) {
                const int e = 64 * i + lane, r = e / (K / 128);
                if (e < ns)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(smem + L.xs + 256 * i), 4,
                                                             (uint32_t)(r * ldxs + 4 * (e - r * (K / 128))), 0, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // The ring's registers and its first loads. NT >= 4: per tile, decode step i's block,
    // then reload the same registers with step i+1's block, so the next step's NT blocks
    // are in flight during this step's decodes while only one block per tile is held (the
    // activation fragments keep a ring of two). With four tiles that is a step of prefetch
    // distance in half the registers of a two-step ring (occupancy 3 instead of 2,
    // measured faster); with fewer tiles the distance gets too short and the two-step
    // ring (step i+1's blocks and activations load while step i decodes) is used.
    constexpr bool kReload = NT >= 4;
    constexpr int kWSteps = kReload ? 1 : kDepth - 1; // steps loaded ahead of the loop
    WTile wr[kReload ? 1 : kDepth][NT];
    ADense ar[kLdsAct ? 1 : (kReload ? 2 : kDepth)][MC];
    // (a wave without blocks loads block b_begin, unused, so every wave issues the same
    // number of loads after its copies)
#pragma unroll
    for (int j = 0; j < kWSteps; ++j) {
        const int blk = count > 0 ? min(first + j * W, last) : b_begin;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            wr[j][nt] = load_w_rsrc(wt[nt], (uint32_t)blk * kTileBytes, lane, col);
        if constexpr (!kLdsAct)
            load_acts(ar[j], blk);
    }
    __builtin_amdgcn_sched_barrier(0);
    // this wave's copies are done once at most its kWLoads * NT * kWSteps weight loads
    // (issued after them) are outstanding
    constexpr int kVm = kWLoads * NT * kWSteps;
    static_assert(kVm < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((kVm & 15) | (7 << 4) | (15 << 8) | ((kVm >> 4) << 14));
    __syncthreads();

    float acc[NT][MC][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int u = 0; u < MC; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[nt][u][r] = 0.0f;
    if (count > 0) {
        if constexpr (kReload) {
            for (int i0 = 0; i0 < count; i0 += 2) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int i = i0 + j;
                    const int bn = min(first + (i + 1) * W, last);
                    if constexpr (!kLdsAct)
                        load_acts(ar[j ^ 1], bn);
                    else
                        load_acts(ar[0], min(first + i * W, last));
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        if constexpr (MAMBO_SCHED_FENCE)
                            __builtin_amdgcn_sched_barrier(0);
                        compute_dense<MC>(wr[0][nt], ar[kLdsAct ? 0 : j], lvl, s_split, acc[nt], i < count);
                        wr[0][nt] = load_w_rsrc(wt[nt], (uint32_t)bn * kTileBytes, lane, col);
                    }
                    if constexpr (MAMBO_SCHED_FENCE)
                        __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else {
            for (int i0 = 0; i0 < count; i0 += kDepth) {
#pragma unroll
                for (int j = 0; j < kDepth; ++j) {
                    const int i = i0 + j;
                    const int slot = (j + kDepth - 1) % kDepth;
                    const int bp = min(first + (i + kDepth - 1) * W, last);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        wr[slot][nt] = load_w_rsrc(wt[nt], (uint32_t)bp * kTileBytes, lane, col);
                    if constexpr (!kLdsAct)
                        load_acts(ar[slot], bp);
                    if constexpr (MAMBO_SCHED_FENCE)
                        __builtin_amdgcn_sched_barrier(0);
                    if constexpr (kLdsAct)
                        load_acts(ar[0], min(first + i * W, last));
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        compute_dense<MC>(wr[j][nt], ar[kLdsAct ? 0 : j], lvl, s_split, acc[nt], i < count);
                    if constexpr (MAMBO_SCHED_FENCE)
                        __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }

#undef load_acts

    // D[i][j] of the MFMA sits in lane j + 16*(i/4), register i%4: token 16u + 4q + r,
    // weight row col. The waves hold partial sums over disjoint K blocks.
    if constexpr (W > 1) {
        float *red = reinterpret_cast<float *>(smem + L.red);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int u = 0; u < MC; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    red[(((wave * NT + nt) * MC + u) * 4 + r) * 64 + lane] = acc[nt][u][r];
        __syncthreads();
        if (wave != 0)
            return;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int u = 0; u < MC; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = 0.0f;
#pragma unroll
                    for (int w = 0; w < W; ++w)
                        v += red[(((w * NT + nt) * MC + u) * 4 + r) * 64 + lane];
                    acc[nt][u][r] = v;
                }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int64_t n = (wg * NT + nt) * kTileRows + col;
#pragma unroll
        for (int u = 0; u < MC; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + 16 * u + 4 * q + r;
                if (m < M && n < N) {
                    float *o = out + m * ldo + n;
                    if (atomic)
                        atomicAdd(o, acc[nt][u][r]);
                    else
                        *o = acc[nt][u][r];
                }
            }
    }
}

// ============================================================================ tiled kernel
// Large M (prefill). A workgroup of W waves computes a 16*MT (tokens) x 16*NT*W (weight
// rows) output tile over all of K. Per 256-weight block the activations of the tile's
// tokens (16*MT rows x 256 bytes + 8 E8M0 scales each) are copied from global memory
// straight into LDS (global_load_lds: no staging registers, no LDS store instructions),
// double buffered in two static arrays; within a row, 16-byte chunk c sits at slot
// c ^ (row & 15), so the 16 rows that one lane group reads fall in 16 different bank
// groups. Each wave decodes its NT weight tiles once per block into dense hi/lo operands
// (as the dense kernel does) and reuses them for all MT token sub-tiles: MT*NT*4 MFMAs
// per block and wave, the fp16 d applied per block in f32. The grid's x runs over
// weight-row tiles (grouped projections start on a workgroup boundary), y over token
// tiles, z over K splits.

// LDS image of one staged block: values [16*MT][256] (chunk-swizzled), scales [16*MT][8].
template <int MT>
struct TiledBlock {
    static constexpr int kRows = 16 * MT;
    static constexpr int kValues = kRows * 256;
    static constexpr int kBytes = kValues + kRows * 8;
};


// Issue the copies of block b's activations into `buf` (buffer loads straight to LDS over
// resources at the tile's first token row): one 1 KiB copy (4 rows, 16 bytes per lane)
// per values instruction and one 256-byte copy (32 rows of scales, 4 bytes per lane) per
// scale instruction, spread over the waves. Rows past M read row M-1 (their outputs are
// never stored). Completion is awaited by the next workgroup barrier.
template <int MT, int W>
__device__ __forceinline__ void stage_block(uint8_t *buf, __amdgpu_buffer_rsrc_t xrows, uint32_t ldxv,
                                            __amdgpu_buffer_rsrc_t srows, uint32_t ldxs, int last_row, int b, int wave,
                                            int lane)
{
    constexpr int kRows = TiledBlock<MT>::kRows;
    constexpr int kVInst = kRows / 4;
    static_assert(kVInst % W == 0, "values copies must spread evenly over the waves");
#pragma unroll
    for (int j = 0; j < kVInst / W; ++j) {
        const int i = wave + j * W;
        const int row = 4 * i + (lane >> 4);
        const uint32_t c = (uint32_t)((lane & 15) ^ (row & 15));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xrows, (lds_ptr)(buf + 1024 * i), 16,
                                                 (uint32_t)min(row, last_row) * ldxv + 16u * c, 256u * b, 0, 0);
    }
    constexpr int kSInst = (kRows + 31) / 32; // a 16-row tile copies its scales with half the lanes
    for (int i = wave; i < kSInst; i += W) {
        const int row = 32 * i + (lane >> 1);
        if (kRows >= 32 || lane < 2 * kRows)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(srows, (lds_ptr)(buf + TiledBlock<MT>::kValues + 256 * i), 4,
                                                     (uint32_t)min(row, last_row) * ldxs + 4u * (lane & 1), 8u * b, 0,
                                                     0);
    }
}

// Decoded dense operands of NT weight tiles for one block (see the dense kernel).
template <int NT>
__device__ __forceinline__ void decode_tiles(const WTile (&w)[NT], const uint8_t *lvl, const uint4 *split,
                                             v8i (&bh)[NT][2], v8i (&bl)[NT][2], float (&d)[NT])
{
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        decode_block(w[nt], lvl, split, bh[nt], bl[nt]);
        d[nt] = half_bits_to_float((uint16_t)w[nt].dh);
    }
}

// MT x NT sub-tiles of one block: A fragments from the staged block (ao: this lane's byte
// offsets of its two 16-byte pieces per K half inside a 16-row sub-tile, soff: its scale
// offset), one chain of four MFMAs (K halves x hi/lo) per sub-tile, then the block's d in
// f32. The fence per sub-tile keeps the compiler from hoisting every LDS read of the
// block into registers.
template <int MT, int NT>
__device__ __forceinline__ void mfma_block(const uint8_t *buf, const uint32_t (&ao)[2][2], uint32_t soff,
                                           const v8i (&bh)[NT][2], const v8i (&bl)[NT][2], const float (&d)[NT],
                                           float (&acc)[MT][NT][4])
{
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const uint8_t *ar = buf + 4096 * mt;
        const uint8_t *sr = buf + TiledBlock<MT>::kValues + 128 * mt + soff;
        v8i av[2];
        int sc[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 lo = *reinterpret_cast<const uint4 *>(ar + ao[h][0]);
            const uint4 hi = *reinterpret_cast<const uint4 *>(ar + ao[h][1]);
            av[h] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            sc[h] = sr[h];
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
            v4f c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[0], bh[nt][0], zero, 0, 0, 0, sc[0], 0, 128);
            c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[0], bl[nt][0], c, 0, 0, 0, sc[0], 0, 128);
            c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[1], bh[nt][1], c, 0, 0, 0, sc[1], 0, 128);
            c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[1], bl[nt][1], c, 0, 0, 0, sc[1], 0, 128);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mt][nt][r] = __builtin_fmaf(c[r], d[nt], acc[mt][nt][r]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Half-K form (the 256 x 256 x 16-wave tile, where the full-K form spills): per block,
// decode K half 0 of the NT weight tiles, run its MFMAs for all MT sub-tiles, then half
// 1; the decoded operands of one half and the block's weight registers (reloaded with
// block b+1 right after their last decode) are all that is held, 128 VGPRs for 16
// sub-tiles of accumulators. d is applied per half (acc += d*c0; acc += d*c1).
template <int NT, int H>
__device__ __forceinline__ void decode_half(const WTile (&w)[NT], const uint8_t *lvl, const uint4 *split,
                                            v8i (&bh)[NT], v8i (&bl)[NT])
{
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t s5[5] = {w[nt].ia.x, w[nt].ia.y, w[nt].ia.z, w[nt].ia.w, (uint32_t)w[nt].ib};
        const uint32_t sc = dense_scales(w[nt].sc);
        decode_split<H>(s5, H == 0 ? w[nt].sg.x : w[nt].sg.y, lvl, split_entry<H, 0>(split, sc),
                        split_entry<H, 1>(split, sc), bh[nt], bl[nt], std::make_integer_sequence<int, 8>{});
    }
}

template <int MT, int NT, int H>
__device__ __forceinline__ void mfma_half(const uint8_t *buf, const uint32_t (&ao)[2][2], uint32_t soff,
                                          const v8i (&bh)[NT], const v8i (&bl)[NT], const float (&d)[NT],
                                          float (&acc)[MT][NT][4])
{
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const uint8_t *ar = buf + 4096 * mt;
        const uint8_t *sr = buf + TiledBlock<MT>::kValues + 128 * mt + soff;
        const uint4 lo = *reinterpret_cast<const uint4 *>(ar + ao[H][0]);
        const uint4 hi = *reinterpret_cast<const uint4 *>(ar + ao[H][1]);
        const v8i av = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        const int sc = sr[H];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
            v4f c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bh[nt], zero, 0, 0, 0, sc, 0, 128);
            c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bl[nt], c, 0, 0, 0, sc, 0, 128);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mt][nt][r] = __builtin_fmaf(c[r], d[nt], acc[mt][nt][r]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// kKs > 1 (16- and 32-token tiles): the W waves form kKs groups of W/kKs that take the
// workgroup's K blocks in turn (group g: blocks b0+g, b0+g+kKs, ...), each group staging
// its own block per step, so a workgroup of the same weight rows holds kKs times the
// waves; the groups' sums are added through LDS in group order at the end.
template <int MT, int NT, int W, bool kHalf = false, int kKs = 1>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2))) void gemm_tiled_kernel(
    const uint8_t *__restrict__ xv, int64_t ldxv,
                                                            const uint8_t *__restrict__ xs, int64_t ldxs, int64_t M,
                                                            GroupArgs ga, int B, int bps, int atomic)
{
    constexpr int kRows = TiledBlock<MT>::kRows;
    constexpr int kThreads = W * 64;
    constexpr int kTw = W / kKs; // waves of one K group (one per NT weight tiles)
    static_assert(W % kKs == 0 && (kKs == 1 || !kHalf), "K groups");
    // a 16-token tile reads each weight once per launch: stream it (non-temporal), as the
    // decode kernels do; larger token tiles re-read it once per token tile
    constexpr int kPolicy = MT == 1 ? kStreamPolicy : 0;
    __shared__ __align__(16) uint8_t s_buf0[kKs * TiledBlock<MT>::kBytes];
    __shared__ __align__(16) uint8_t s_buf1[kKs * TiledBlock<MT>::kBytes];
    __shared__ uint32_t s_lvl[512];
    __shared__ uint4 s_split[16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = kKs == 1 ? 0 : wave_all / kTw;  // K group
    const int wave = wave_all - kg * kTw;           // wave within the group
    const int col = lane & 15, q = lane >> 4;

    // this workgroup's projection; tile_begin counts workgroups here
    const uint8_t *packed = ga.packed[0];
    float *out = ga.out[0];
    int64_t N = ga.n[0], ldo = ga.ldo[0], wg = blockIdx.x;
#pragma unroll
    for (int g = 1; g < kMaxGroup; ++g)
        if (g < ga.count && (int64_t)blockIdx.x >= ga.tile_begin[g]) {
            packed = ga.packed[g];
            out = ga.out[g];
            N = ga.n[g];
            ldo = ga.ldo[g];
            wg = blockIdx.x - ga.tile_begin[g];
        }
    const int64_t tiles = (N + kTileRows - 1) / kTileRows;
    const int64_t m0 = (int64_t)blockIdx.y * kRows;
    // weight tiles of this wave (clamped to the last tile; stores are masked)
    __amdgpu_buffer_rsrc_t wt[NT];
    int64_t tile[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        tile[nt] = wg * (NT * kTw) + wave * NT + nt;
        wt[nt] = byte_rsrc(packed + min(tile[nt], tiles - 1) * (int64_t)B * kTileBytes);
    }

    for (int i = tid; i < 512; i += kThreads)
        s_lvl[i] = c_grid.level[i];
    if (tid < 16)
        s_split[tid] = uint4{c_split.w[tid][0], c_split.w[tid][1], c_split.w[tid][2], c_split.w[tid][3]};

    const __amdgpu_buffer_rsrc_t xrows = byte_rsrc(xv + m0 * ldxv), srows = byte_rsrc(xs + m0 * ldxs);
    const int last_row = (int)min<int64_t>(M - 1 - m0, kRows - 1);
    // A operand of lane (token row col of a sub-tile, q): per K half h the 16-byte chunks
    // c = 8*(q>>1) + (q&1) + 2h and c + 4 of the row (see the dense kernel for the byte and
    // scale order), at their swizzled slots; scale byte 4*(q&1) + 2*(q>>1) + h.
    uint32_t ao[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int p = 0; p < 2; ++p)
            ao[h][p] = 256u * col + 16u * ((8u * (q >> 1) + (q & 1) + 2u * h + 4u * p) ^ (uint32_t)col);
    const uint32_t soff = 8u * col + 4u * (q & 1) + 2u * (q >> 1);

    float acc[MT][NT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[mt][nt][r] = 0.0f;

    // K range of this workgroup: blocks [b0, b1) (grid z splits K; partial sums are
    // added into an output zeroed beforehand). Step s: K group kg takes block
    // b0 + s*kKs + kg (clamped for its loads; no math past b1).
    const uint8_t *lvl = reinterpret_cast<const uint8_t *>(s_lvl);
    const int b0 = blockIdx.z * bps, b1 = min(B, b0 + bps);
    WTile wcur[NT], wnext[kHalf ? 1 : NT];
    v8i bh[kHalf ? 1 : NT][2], bl[kHalf ? 1 : NT][2]; // full-K form
    v8i hh[NT], hl[NT];                              // half-K form
    float d[NT];
    constexpr int kBufStride = TiledBlock<MT>::kBytes;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
        wcur[nt] = load_w_rsrc<kPolicy>(wt[nt], (uint32_t)min(b0 + kg, b1 - 1) * kTileBytes, lane, col);
    stage_block<MT, kTw>(s_buf0 + kg * kBufStride, xrows, (uint32_t)ldxv, srows, (uint32_t)ldxs, last_row,
                         min(b0 + kg, b1 - 1), wave, lane);
    __syncthreads();

    // Block b: copy block b+1's activations into the other buffer and request its weight
    // tiles, then decode block b's weights and run its MFMAs; the barrier at the end waits
    // for the copies (and frees this buffer for block b+2's). Two fixed buffers (the loop
    // is unrolled by two), so the compiler can tell the copy target from the buffer read.
    // (b: this K group's block of the step; b + kKs: its next one.)
#define MAMBO_TILED_BLOCK(cur_, nxt_)                                                                              \
    do {                                                                                                           \
        uint8_t *cur = (cur_) + kg * kBufStride;                                                                   \
        uint8_t *nxt = (nxt_) + kg * kBufStride;                                                                   \
        stage_block<MT, kTw>(nxt, xrows, (uint32_t)ldxv, srows, (uint32_t)ldxs, last_row, min(b + kKs, b1 - 1),     \
                             wave, lane);                                                                          \
        const uint32_t next_ = (uint32_t)min(b + kKs, b1 - 1) * kTileBytes;                                        \
        if constexpr (kHalf) {                                                                                     \
            __builtin_amdgcn_sched_barrier(0);                                                                     \
            for (int nt = 0; nt < NT; ++nt)                                                                        \
                d[nt] = half_bits_to_float((uint16_t)wcur[nt].dh);                                                 \
            decode_half<NT, 0>(wcur, lvl, s_split, hh, hl);                                                        \
            mfma_half<MT, NT, 0>(cur, ao, soff, hh, hl, d, acc);                                                   \
            decode_half<NT, 1>(wcur, lvl, s_split, hh, hl);                                                        \
            for (int nt = 0; nt < NT; ++nt)                                                                        \
                wcur[nt] = load_w_rsrc<kPolicy>(wt[nt], next_, lane, col);                                         \
            mfma_half<MT, NT, 1>(cur, ao, soff, hh, hl, d, acc);                                                   \
        } else {                                                                                                   \
            for (int nt = 0; nt < NT; ++nt)                                                                        \
                wnext[nt] = load_w_rsrc<kPolicy>(wt[nt], next_, lane, col);                                        \
            __builtin_amdgcn_sched_barrier(0);                                                                     \
            if (kKs == 1 || b < b1) {                                                                              \
                decode_tiles<NT>(wcur, lvl, s_split, bh, bl, d);                                                   \
                mfma_block<MT, NT>(cur, ao, soff, bh, bl, d, acc);                                                 \
            }                                                                                                      \
            for (int nt = 0; nt < NT; ++nt)                                                                        \
                wcur[nt] = wnext[nt];                                                                              \
        }                                                                                                          \
        __syncthreads();                                                                                           \
    } while (0)
    // steps: the same count for every K group (a group past b1 only stages and waits)
    const int b_end = b0 + (b1 - b0 + kKs - 1) / kKs * kKs;
    for (int b = b0 + kg; b < b_end; b += kKs) {
        MAMBO_TILED_BLOCK(s_buf0, s_buf1);
        if ((b += kKs) >= b_end)
            break;
        MAMBO_TILED_BLOCK(s_buf1, s_buf0);
    }
#undef MAMBO_TILED_BLOCK
    if constexpr (kKs > 1) {
        // groups 1.. hand their sums to group 0 through LDS (the loop's last barrier has
        // retired every copy into the buffers); group 0 adds them in group order
        constexpr int kE = MT * NT * 4;
        static_assert((kKs - 1) * kTw * 64 * kE * 4 <= kKs * TiledBlock<MT>::kBytes, "reduction fits buffer 0");
        float *red = reinterpret_cast<float *>(s_buf0);
        if (kg > 0) {
            float *dst = red + ((kg - 1) * kTw + wave) * 64 * kE + lane;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        dst[64 * ((mt * NT + nt) * 4 + r)] = acc[mt][nt][r];
        }
        __syncthreads();
        if (kg > 0)
            return;
#pragma unroll
        for (int g = 1; g < kKs; ++g) {
            const float *src = red + ((g - 1) * kTw + wave) * 64 * kE + lane;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[mt][nt][r] += src[64 * ((mt * NT + nt) * 4 + r)];
        }
    }

    // D[i][j] of sub-tile (mt, nt): lane j + 16*(i/4), register i%4 -> token
    // m0 + 16*mt + 4q + r, weight row 16*tile + col. The lane's col and q are recomputed
    // here from the lane count (v_mbcnt) rather than kept from the thread id across the
    // block loop: in the 256 x 256 x 16 tile (128 VGPRs) keeping them spilled two
    // registers, and a kernel with spills takes scratch memory at every dispatch.
    const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int col_e = lane_e & 15, q_e = lane_e >> 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int64_t n = tile[nt] * kTileRows + col_e;
        if (n >= N)
            continue;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + 16 * mt + 4 * q_e + r;
                if (m < M) {
                    if (atomic)
                        atomicAdd(out + m * ldo + n, acc[mt][nt][r]);
                    else
                        __builtin_nontemporal_store(acc[mt][nt][r], out + m * ldo + n); // written once
                }
            }
    }
}

// ---------------------------------------------------------------------------- prefill form
// 256 tokens x 16*W weight rows (W waves of 16 rows, one workgroup per CU), with the
// decode of block b+1 spread over the MFMAs of block b inside each wave:
//  * step mt (mt = 0..15) of block b: the four MFMAs of 16-token sub-tile mt (K halves x
//    hi/lo, one accumulator chain), then the activation fragments and scales of sub-tile
//    mt+1 are requested, the codebook word of code mt of block b+1 is requested and code
//    mt-1 is finished (two perms, two sign ops), and sub-tile mt-1's result is scaled by
//    d into its accumulators. Every wait is for something requested a step earlier (about
//    128 MFMA cycles), and each step issues ~12 VALU instructions against four MFMAs.
//  * the decoded operands of two blocks (current and next, 2 x 32 VGPRs) and the packed
//    weights of the next two blocks are held: block b issues the copies of block b+1's
//    activations, then the loads of block b+2's weights, so every wait is partial (the
//    decode waits for loads issued a block earlier, the barrier for the copies only);
//    the block loop is unrolled by two so the operand sets swap without moves.
//  * each lane reads both activation scale bytes of a sub-tile with one 16-bit load and
//    the MFMA picks byte h with op_sel; the codebook, the split table and the scale
//    buffers lie below 64 KiB of LDS so their addresses fold into the offset field.
// 2 waves per SIMD at W = 8 (256 VGPRs per wave).
// LDS of the prefill form: one __shared__ array per buffer, so the compiler can tell the
// copy target (buffer C^1) from the buffer being read (C) and does not wait for the copies
// before reading; the tables and scale buffers are declared first and land below 64 KiB.
struct PrefillLds {
    static constexpr int kRows = 256;
};

// Decoded operands of one 16-row weight tile for one block, in the dense K order.
struct Decoded {
    v8i hi[2], lo[2];
    float d;
};

// Per-code pieces of the decode (decode_split split into steps). Code I (0..15) is code
// I % 8 of MFMA I / 8; codes 4k .. 4k+3 use split-table entry k, which the fetch of code
// 4k reads into slot k & 1 (the finish of code 4k-1, one step behind, still reads the
// other slot), so only two entries are held.
struct DecodeState {
    uint32_t s[5];   // index bit stream
    uint32_t p[2];   // transposed sign words of the lane's two halves
    uint32_t sc;     // scale nibbles (dense_scales)
    uint4 tab[2];    // split-table entries in use
    float d;         // the row's d in f32
};

__device__ __forceinline__ void decode_begin(DecodeState &st, const WTile &w)
{
    st.s[0] = w.ia.x;
    st.s[1] = w.ia.y;
    st.s[2] = w.ia.z;
    st.s[3] = w.ia.w;
    st.s[4] = (uint32_t)w.ib;
    st.p[0] = w.sg.x;
    st.p[1] = w.sg.y;
    st.sc = dense_scales(w.sc);
    // d becomes an f32 register here, where the decode waits for this block's weights
    // anyway. Left as the raw fp16 word, the compiler folded the conversion into the
    // post-scale (v_fma_mix) and carried the word of the block two ahead across the loop
    // back edge with a register copy that waited for every load in flight (vmcnt 0).
    float d = half_bits_to_float(w.dh);
    asm volatile("" : "+v"(d));
    st.d = d;
}

template <int I>
__device__ __forceinline__ uint32_t decode_fetch(DecodeState &st, const uint8_t *lvl, const uint4 *split)
{
    if constexpr (I % 4 == 0)
        st.tab[(I / 4) & 1] = split_entry<I / 8, (I / 4) & 1>(split, st.sc);
    return *reinterpret_cast<const uint32_t *>(lvl + code_addr<I>(st.s));
}

template <int I>
__device__ __forceinline__ void decode_finish(const DecodeState &st, uint32_t lv, Decoded &out)
{
    constexpr int H = I / 8, C = I % 8;
    int hi, lo;
    split_word<C>(lv, st.p[H], st.tab[(I / 4) & 1], hi, lo);
    out.hi[H][C] = hi;
    out.lo[H][C] = lo;
}

// Copies of block b's activations into one buffer of the prefill LDS (values `vals`, scales
// `scl`): value copy j of a wave moves 4 rows (1 KiB, offsets voff[j]), waves 0..7 one
// scale copy each.
template <int W>
__device__ __forceinline__ void prefill_stage(uint8_t *vals, uint8_t *scl, int b, __amdgpu_buffer_rsrc_t xrows,
                                              __amdgpu_buffer_rsrc_t srows, const uint32_t (&voff)[256 / 4 / W],
                                              uint32_t soff_stage, int wave)
{
#pragma unroll
    for (int j = 0; j < 256 / 4 / W; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xrows, (lds_ptr)(vals + 1024 * (wave + W * j)), 16, voff[j], 256u * b,
                                                 0, 0);
    if (wave < PrefillLds::kRows / 32)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(srows, (lds_ptr)(scl + 256 * wave), 4, soff_stage, 8u * b, 0, 0);
}

// Sub-tiles whose activation fragments are requested ahead of their MFMAs.
#ifndef MAMBO_PREFILL_AHEAD
#define MAMBO_PREFILL_AHEAD 2
#endif
constexpr int kPrefillAhead = MAMBO_PREFILL_AHEAD;

// Operands of one prefill block in flight: activation fragments and scales of
// kPrefillAhead + 1 sub-tiles (slots), codebook words of two codes, the previous
// sub-tile's result.
struct PrefillPipe {
    v8i a[kPrefillAhead + 1][2];
    int sc[kPrefillAhead + 1];
    uint32_t lw[2];
    v4f prev;
};

__device__ __forceinline__ void prefill_load(PrefillPipe &pp, int slot, const uint8_t *ar, const uint32_t (&ao)[2][2],
                                             const uint8_t *sr)
{
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4 lo = *reinterpret_cast<const uint4 *>(ar + ao[h][0]);
        const uint4 hi = *reinterpret_cast<const uint4 *>(ar + ao[h][1]);
        pp.a[slot][h] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
    pp.sc[slot] = (int)*reinterpret_cast<const uint16_t *>(sr);
}

// Step mt of a prefill block (see gemm_prefill_kernel): sub-tile mt's MFMAs with operands
// `cur`, the next sub-tile's loads, code mt of the next block's decode requested and code
// mt-1 finished into `nxt`, sub-tile mt-1 scaled into its accumulators.
template <int mt>
__device__ __forceinline__ void prefill_step(PrefillPipe &pp, const Decoded &cur, Decoded &nxt, DecodeState &st,
                                             const uint8_t *vals, const uint8_t *scl, const uint32_t (&ao)[2][2],
                                             uint32_t soff, const uint8_t *lvl, const uint4 *split, float d,
                                             float (&acc)[16][4])
{
    constexpr int sl = mt % (kPrefillAhead + 1), cw = mt & 1;
    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(pp.a[sl][0], cur.hi[0], zero, 0, 0, 0, pp.sc[sl], 0, 128);
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(pp.a[sl][0], cur.lo[0], c, 0, 0, 0, pp.sc[sl], 0, 128);
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(pp.a[sl][1], cur.hi[1], c, 0, 0, 1, pp.sc[sl], 0, 128);
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(pp.a[sl][1], cur.lo[1], c, 0, 0, 1, pp.sc[sl], 0, 128);
    if constexpr (mt + kPrefillAhead < 16)
        prefill_load(pp, (mt + kPrefillAhead) % (kPrefillAhead + 1), vals + 4096 * (mt + kPrefillAhead), ao,
                     scl + 128 * (mt + kPrefillAhead) + soff);
    pp.lw[cw] = decode_fetch<mt>(st, lvl, split);
    if constexpr (mt > 0) {
        decode_finish<mt - 1>(st, pp.lw[cw ^ 1], nxt);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[mt - 1][r] = __builtin_fmaf(pp.prev[r], d, acc[mt - 1][r]);
    }
    pp.prev = c;
    __builtin_amdgcn_sched_barrier(0);
}

template <int... MT>
__device__ __forceinline__ void prefill_steps(PrefillPipe &pp, const Decoded &cur, Decoded &nxt, DecodeState &st,
                                              const uint8_t *vals, const uint8_t *scl, const uint32_t (&ao)[2][2],
                                              uint32_t soff, const uint8_t *lvl, const uint4 *split, float d,
                                              float (&acc)[16][4], std::integer_sequence<int, MT...>)
{
    (prefill_step<MT>(pp, cur, nxt, st, vals, scl, ao, soff, lvl, split, d, acc), ...);
}

template <int... I>
__device__ __forceinline__ void decode_all(DecodeState &st, const uint8_t *lvl, const uint4 *split, Decoded &out,
                                           std::integer_sequence<int, I...>)
{
    ((decode_finish<I>(st, decode_fetch<I>(st, lvl, split), out)), ...);
}

template <int W>
__global__ __launch_bounds__(W * 64) void gemm_prefill_kernel(const uint8_t *__restrict__ xv, int64_t ldxv,
                                                              const uint8_t *__restrict__ xs, int64_t ldxs, int64_t M,
                                                              GroupArgs ga, int B, int bps, int atomic)
{
    using L = PrefillLds;
    constexpr int kRows = L::kRows;
    constexpr int kThreads = W * 64;
    constexpr int kVCopies = kRows / 4 / W;   // 1 KiB value copies per wave and block
    constexpr int kSCopies = kRows / 32;      // 256-byte scale copies per block (waves 0..kSCopies-1)
    static_assert(kRows / 4 % W == 0 && kSCopies <= W, "staging must spread evenly over the waves");
    __shared__ uint32_t s_lvl[512];
    __shared__ uint4 s_split[16];
    __shared__ __align__(16) uint8_t s_scale0[kRows * 8];
    __shared__ __align__(16) uint8_t s_scale1[kRows * 8];
    __shared__ __align__(16) uint8_t s_vals0[kRows * 256];
    __shared__ __align__(16) uint8_t s_vals1[kRows * 256];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, q = lane >> 4;

    const uint8_t *packed = ga.packed[0];
    float *out = ga.out[0];
    int64_t N = ga.n[0], ldo = ga.ldo[0], wg = blockIdx.x;
#pragma unroll
    for (int g = 1; g < kMaxGroup; ++g)
        if (g < ga.count && (int64_t)blockIdx.x >= ga.tile_begin[g]) {
            packed = ga.packed[g];
            out = ga.out[g];
            N = ga.n[g];
            ldo = ga.ldo[g];
            wg = blockIdx.x - ga.tile_begin[g];
        }
    const int64_t tiles = (N + kTileRows - 1) / kTileRows;
    const int64_t m0 = (int64_t)blockIdx.y * kRows;
    const int64_t tile = wg * W + wave;
    const __amdgpu_buffer_rsrc_t wt = byte_rsrc(packed + min(tile, tiles - 1) * (int64_t)B * kTileBytes);

    for (int i = tid; i < 512; i += kThreads)
        s_lvl[i] = c_grid.level[i];
    if (tid < 16)
        s_split[tid] = uint4{c_split.w[tid][0], c_split.w[tid][1], c_split.w[tid][2], c_split.w[tid][3]};

    // Staging: value copy j of this wave moves rows 4*(wave + W*j) .. +3 (16 bytes per
    // lane, chunk slot lane&15 of row r holds source chunk (lane&15) ^ (r&15)); rows past M
    // read row M-1. Offsets are loop-invariant; the block offset goes in the scalar offset.
    const __amdgpu_buffer_rsrc_t xrows = byte_rsrc(xv + m0 * ldxv), srows = byte_rsrc(xs + m0 * ldxs);
    const int last_row = (int)min<int64_t>(M - 1 - m0, kRows - 1);
    uint32_t voff[kVCopies];
#pragma unroll
    for (int j = 0; j < kVCopies; ++j) {
        const int row = 4 * (wave + W * j) + (lane >> 4);
        voff[j] = (uint32_t)min(row, last_row) * (uint32_t)ldxv + 16u * (uint32_t)((lane & 15) ^ (row & 15));
    }
    // Offset of this lane's scale copy: recomputed per block from a lane id the compiler
    // cannot see through (three VALU instructions). Hoisted out of the loop it was the
    // register spilled at 256 VGPRs, and its reload (a scratch load, counted with the
    // weight loads) made every block wait for all loads in flight before its copies.
    auto stage_soff = [&]() {
        uint32_t l = (uint32_t)lane;
        asm volatile("" : "+v"(l));
        return (uint32_t)min(32 * wave + (int)(l >> 1), last_row) * (uint32_t)ldxs + 4u * (l & 1);
    };

    // A operand of lane (token row col of a sub-tile, q), K half h: 16-byte chunks
    // 8*(q>>1) + (q&1) + 2h and +4 of the row at their swizzled slots (the dense kernel's
    // K order); its scale bytes for h = 0, 1 are adjacent at soff.
    uint32_t ao[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
            ao[h][pp] = 256u * col + 16u * ((8u * (q >> 1) + (q & 1) + 2u * h + 4u * pp) ^ (uint32_t)col);
    const uint32_t soff = 8u * col + 4u * (q & 1) + 2u * (q >> 1);

    float acc[16][4];
#pragma unroll
    for (int mt = 0; mt < 16; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[mt][r] = 0.0f;

    const uint8_t *lvl = reinterpret_cast<const uint8_t *>(s_lvl);
    const int b0 = blockIdx.z * bps, b1 = min(B, b0 + bps);
    auto wblock = [&](int b) { return (uint32_t)min(b, b1 - 1) * kTileBytes; };
    // packed weights: block b0 decoded up front, b0+1 in slot 0; block b requests block
    // b+2's weights into the slot its predecessor decoded from, right after its activation
    // copies (vector memory completes in issue order: the decode waits only for loads a
    // block old, the barrier only for the copies)
    WTile wslot[2];
    Decoded dec[2];
    {
        const WTile w0 = load_w_rsrc<0>(wt, wblock(b0), lane, col);
        wslot[0] = load_w_rsrc<0>(wt, wblock(b0 + 1), lane, col);
        prefill_stage<W>(s_vals0, s_scale0, b0, xrows, srows, voff, stage_soff(), wave);
        __syncthreads(); // codebook and split tables
        DecodeState st;
        decode_begin(st, w0);
        decode_all(st, lvl, s_split, dec[0], std::make_integer_sequence<int, 16>{});
        dec[0].d = st.d;
    }
    __syncthreads();

    // Block b with operands dec[C] (decoding block b+1 from wslot[C] into dec[C^1]);
    // buffer C (= (b - b0) & 1) holds block b's activations. A macro, so C is a constant:
    // the two operand sets are fixed registers and the two buffers fixed arrays.
#define MAMBO_PREFILL_BLOCK(C)                                                                                     \
    do {                                                                                                           \
        const uint8_t *vals_ = (C) ? s_vals1 : s_vals0;                                                            \
        const uint8_t *scl_ = (C) ? s_scale1 : s_scale0;                                                           \
        prefill_stage<W>((C) ? s_vals0 : s_vals1, (C) ? s_scale0 : s_scale1, min(b + 1, b1 - 1), xrows, srows,     \
                         voff, stage_soff(), wave);                                                                \
        wslot[(C) ^ 1] = load_w_rsrc<0>(wt, wblock(b + 2), lane, col);                                             \
        DecodeState st_;                                                                                           \
        decode_begin(st_, wslot[C]);                                                                               \
        PrefillPipe pp_;                                                                                           \
        for (int t_ = 0; t_ < kPrefillAhead; ++t_)                                                                 \
            prefill_load(pp_, t_, vals_ + 4096 * t_, ao, scl_ + 128 * t_ + soff);                                  \
        prefill_steps(pp_, dec[C], dec[(C) ^ 1], st_, vals_, scl_, ao, soff, lvl, s_split, dec[C].d, acc,          \
                      std::make_integer_sequence<int, 16>{});                                                      \
        decode_finish<15>(st_, pp_.lw[1], dec[(C) ^ 1]);                                                           \
        dec[(C) ^ 1].d = st_.d;                                                                                    \
        for (int r = 0; r < 4; ++r)                                                                                \
            acc[15][r] = __builtin_fmaf(pp_.prev[r], dec[C].d, acc[15][r]);                                        \
        __syncthreads();                                                                                           \
    } while (0)
    for (int b = b0; b < b1; ++b) {
        MAMBO_PREFILL_BLOCK(0);
        if (++b == b1)
            break;
        MAMBO_PREFILL_BLOCK(1);
    }
#undef MAMBO_PREFILL_BLOCK

    const int64_t n = tile * kTileRows + col;
    if (n < N) {
#pragma unroll
        for (int mt = 0; mt < 16; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + 16 * mt + 4 * q + r;
                if (m < M) {
                    if (atomic)
                        atomicAdd(out + m * ldo + n, acc[mt][r]);
                    else
                        __builtin_nontemporal_store(acc[mt][r], out + m * ldo + n); // written once
                }
            }
    }
}

// Zero rows [0, M) of projection blockIdx.y's output (the split-K accumulators of every
// projection of a launch in one dispatch): each thread clears a 4-float chunk of a row
// (chunks flattened over rows, grid-strided), with one 16-byte store where the chunk is
// whole and 16-byte aligned (column slices of a wider buffer may not be). The chunk index
// is 64-bit: the grid stride (up to 1024 x 256) added to an index near the end of a large
// output must not wrap. The projection is picked by selects over constant indices, so the
// arguments stay in scalar registers.
__global__ __launch_bounds__(256) void zero_rows_kernel(GroupArgs ga, int M)
{
    const int g = blockIdx.y;
    float *out = ga.out[0];
    int64_t cols = ga.n[0], ld = ga.ldo[0];
#pragma unroll
    for (int i = 1; i < kMaxGroup; ++i)
        if (g == i) {
            out = ga.out[i];
            cols = ga.n[i];
            ld = ga.ldo[i];
        }
    const int64_t chunks = (cols + 3) / 4;
    const int64_t total = (int64_t)M * chunks;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / chunks, c = 4 * (i - r * chunks);
        float *p = out + r * ld + c;
        if (c + 4 <= cols && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
            __builtin_nontemporal_store(v4f{0.0f, 0.0f, 0.0f, 0.0f}, reinterpret_cast<v4f *>(p));
        } else {
            for (int64_t j = c; j < cols && j < c + 4; ++j)
                __builtin_nontemporal_store(0.0f, out + r * ld + j);
        }
    }
}

// Launch arguments of the stream kernel beyond the operands.
struct StreamLaunch {
    dim3 grid;
    size_t lds;
    int64_t ntiles; // 16-row tiles of the launch (all projections)
    int tpw;        // tiles per workgroup
    int B, bps, atomic;
    int lg;         // log2 of the codebook copies (0, 2 or 4; 0 when U > 1)
};

template <int U, int W, bool kLdsAct, int kQ = 0, int kLg = 0>
void launch_stream_uwa(const StreamLaunch &sl, hipStream_t stream, const uint8_t *xv, int64_t ldxv, const uint8_t *xs,
                       int64_t ldxs, int64_t M, const GroupArgs &ga)
{
    MAMBO_LAUNCH((gemm_stream_kernel<U, W, kLdsAct, kQ, kLg>), sl.grid, dim3(W * 64), sl.lds, stream, xv, ldxv, xs,
                       ldxs, M, ga, sl.ntiles, sl.tpw, sl.B, sl.bps, sl.atomic);
}

template <int U, int W, bool kLdsAct, int kQ = 0>
void launch_stream_uwl(const StreamLaunch &sl, hipStream_t stream, const uint8_t *xv, int64_t ldxv, const uint8_t *xs,
                       int64_t ldxs, int64_t M, const GroupArgs &ga)
{
    if constexpr (U == 1) {
        if (sl.lg == 2)
            return launch_stream_uwa<U, W, kLdsAct, kQ, 2>(sl, stream, xv, ldxv, xs, ldxs, M, ga);
        if (sl.lg == 4)
            return launch_stream_uwa<U, W, kLdsAct, kQ, 4>(sl, stream, xv, ldxv, xs, ldxs, M, ga);
    }
    launch_stream_uwa<U, W, kLdsAct, kQ>(sl, stream, xv, ldxv, xs, ldxs, M, ga);
}

// quant: -1 for MXFP8 activations, else the MAMBO_DTYPE_* of unquantized rows that the
// kernel quantizes itself (built for one 4-token sub-tile with LDS-staged rows only).
template <int U, int W>
void launch_stream_uw(bool lds_act, int quant, const StreamLaunch &sl, hipStream_t stream, const uint8_t *xv,
                      int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t M, const GroupArgs &ga)
{
    if constexpr (U == 1) {
        if (quant == MAMBO_DTYPE_BF16)
            return launch_stream_uwl<U, W, true, 1>(sl, stream, xv, ldxv, xs, ldxs, M, ga);
        if (quant == MAMBO_DTYPE_F32)
            return launch_stream_uwl<U, W, true, 2>(sl, stream, xv, ldxv, xs, ldxs, M, ga);
    }
    if (lds_act)
        launch_stream_uwl<U, W, true>(sl, stream, xv, ldxv, xs, ldxs, M, ga);
    else
        launch_stream_uwl<U, W, false>(sl, stream, xv, ldxv, xs, ldxs, M, ga);
}

// Waves per workgroup the stream kernel is built for.
constexpr int kStreamWaves[] = {1, 2, 4, 6, 8, 12, 16};

// dry: check that the configuration is built, launch nothing.
template <int U>
int launch_stream_u(bool dry, int waves, bool lds_act, int quant, const StreamLaunch &sl, hipStream_t stream,
                    const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t M, const GroupArgs &ga)
{
#define MAMBO_W(WV)                                                                                                \
    case WV:                                                                                                       \
        if (!dry)                                                                                                  \
            launch_stream_uw<U, WV>(lds_act, quant, sl, stream, xv, ldxv, xs, ldxs, M, ga);                          \
        break;
    switch (waves) {
        MAMBO_W(1) MAMBO_W(2) MAMBO_W(4) MAMBO_W(6) MAMBO_W(8) MAMBO_W(12) MAMBO_W(16)
    default:
        return mambo_fail(MAMBO_ERR_VALUE, "waves must be one of 1, 2, 4, 6, 8, 12, 16 (got %d)", waves);
    }
#undef MAMBO_W
    return MAMBO_OK;
}

template <int W, int NT, int MC>
void launch_dense_wnm(bool lds_act, dim3 grid, size_t lds, hipStream_t stream, const uint8_t *xv, int64_t ldxv,
                      const uint8_t *xs, int64_t ldxs, int64_t M, const GroupArgs &ga, int B, int bps, int atomic)
{
    if (lds_act)
        MAMBO_LAUNCH((gemm_dense_kernel<W, NT, true, MC>), grid, dim3(W * 64), lds, stream, xv, ldxv, xs, ldxs,
                           M, ga, B, bps, atomic);
    else
        MAMBO_LAUNCH((gemm_dense_kernel<W, NT, false, MC>), grid, dim3(W * 64), lds, stream, xv, ldxv, xs, ldxs,
                           M, ga, B, bps, atomic);
}

template <int NT>
int launch_dense_n(bool dry, int waves, int mc, bool lds_act, dim3 grid, size_t lds, hipStream_t stream,
                   const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t M, const GroupArgs &ga,
                   int B, int bps, int atomic)
{
#define MAMBO_W(WV)                                                                                                \
    case WV:                                                                                                       \
        if (!dry)                                                                                                  \
            launch_dense_wnm<WV, NT, 1>(lds_act, grid, lds, stream, xv, ldxv, xs, ldxs, M, ga, B, bps, atomic);     \
        break;
#define MAMBO_W2(WV)                                                                                               \
    case WV:                                                                                                       \
        if (!dry)                                                                                                  \
            launch_dense_wnm<WV, NT, 2>(lds_act, grid, lds, stream, xv, ldxv, xs, ldxs, M, ga, B, bps, atomic);     \
        break;
    if (mc == 2) {
        switch (waves) {
            MAMBO_W2(2) MAMBO_W2(4) MAMBO_W2(8)
        default:
            return mambo_fail(MAMBO_ERR_VALUE, "dense kernel with tile_m=32: waves must be 2, 4 or 8 (got %d)", waves);
        }
        return MAMBO_OK;
    }
    switch (waves) {
        MAMBO_W(1) MAMBO_W(2) MAMBO_W(4) MAMBO_W(6) MAMBO_W(8) MAMBO_W(12) MAMBO_W(16)
    default:
        return mambo_fail(MAMBO_ERR_VALUE, "waves must be one of 1, 2, 4, 6, 8, 12, 16 (got %d)", waves);
    }
#undef MAMBO_W
#undef MAMBO_W2
    return MAMBO_OK;
}

int launch_dense(bool dry, int waves, int nt, int mc, bool lds_act, dim3 grid, size_t lds, hipStream_t stream,
                 const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t M, const GroupArgs &ga, int B,
                 int bps, int atomic)
{
    switch (nt) {
    case 1: return launch_dense_n<1>(dry, waves, mc, lds_act, grid, lds, stream, xv, ldxv, xs, ldxs, M, ga, B, bps, atomic);
    case 2: return launch_dense_n<2>(dry, waves, mc, lds_act, grid, lds, stream, xv, ldxv, xs, ldxs, M, ga, B, bps, atomic);
    case 4: return launch_dense_n<4>(dry, waves, mc, lds_act, grid, lds, stream, xv, ldxv, xs, ldxs, M, ga, B, bps, atomic);
    default: return mambo_fail(MAMBO_ERR_VALUE, "dense kernel: tile_n must be 16, 32 or 64 (got %d)", 16 * nt);
    }
}

template <int MT, int NT, int W, int KS>
void launch_tiled_t(dim3 grid, hipStream_t stream, const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs,
                    int64_t M, const GroupArgs &ga, int B, int bps, int atomic)
{
    if constexpr (MT >= 16 && NT == 1 && W == 8) // 256 x 128 x 8: the pipelined prefill form
        MAMBO_LAUNCH((gemm_prefill_kernel<W>), grid, dim3(W * 64), 0, stream, xv, ldxv, xs, ldxs, M, ga, B, bps,
                     atomic);
    else // direct copies; the 256-token tiles of 256 weight rows in the half-K form
        MAMBO_LAUNCH((gemm_tiled_kernel<MT, NT, W, (MT >= 16), KS>), grid, dim3(W * 64), 0, stream, xv, ldxv, xs,
                           ldxs, M, ga, B, bps, atomic);
}

// K groups of a tiled configuration: in the 16- and 32-token tiles a K group is the
// waves that cover tile_n weight rows (4 waves of 16 * (tile_n / 64) rows for tile_n >= 64,
// else tile_n / 16 waves of 16 rows), and `waves` beyond one group are further groups
// splitting the workgroup's K blocks (all but the 32-token tile of 8 waves x 16 rows,
// tile_n = 128, which is one group); the larger tiles have one group.
int tiled_groups(const mambo_gemm_config &c)
{
    if (c.tile_m > 32 || (c.tile_m == 32 && c.waves == 8 && c.tile_n == 128))
        return 1;
    const int tw = c.tile_n >= 64 ? 4 : std::max(1, c.tile_n / 16);
    return std::max(1, c.waves / tw);
}

// Tile shapes the tiled kernel is built for: (tokens, weight rows per wave / 16, waves, K
// groups).
int launch_tiled(bool dry, int mt, int nt, int waves, int ks, dim3 grid, hipStream_t stream, const uint8_t *xv,
                 int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t M, const GroupArgs &ga, int B, int bps,
                 int atomic)
{
#define MAMBO_T(A, C, D, E)                                                                                        \
    if (mt == A && nt == C && waves == D && ks == E) {                                                             \
        if (!dry)                                                                                                  \
            launch_tiled_t<A, C, D, E>(grid, stream, xv, ldxv, xs, ldxs, M, ga, B, bps, atomic);                   \
        return MAMBO_OK;                                                                                           \
    }
    MAMBO_T(1, 1, 4, 1) MAMBO_T(1, 2, 4, 1) MAMBO_T(1, 4, 4, 1) MAMBO_T(2, 1, 4, 1) MAMBO_T(2, 2, 4, 1)
    MAMBO_T(2, 1, 8, 1) MAMBO_T(1, 1, 8, 2) MAMBO_T(1, 2, 8, 2) MAMBO_T(1, 1, 16, 4) MAMBO_T(2, 1, 8, 2)
    MAMBO_T(1, 1, 4, 4) MAMBO_T(1, 1, 4, 2) MAMBO_T(1, 1, 8, 8) MAMBO_T(1, 1, 8, 4) MAMBO_T(1, 1, 16, 16)
    MAMBO_T(1, 1, 16, 8) MAMBO_T(2, 1, 8, 8) MAMBO_T(2, 1, 8, 4)
    MAMBO_T(16, 1, 16, 1) MAMBO_T(16, 1, 8, 1) MAMBO_T(8, 2, 8, 1) MAMBO_T(8, 2, 4, 1) MAMBO_T(8, 1, 8, 1)
    MAMBO_T(8, 1, 4, 1) MAMBO_T(4, 2, 8, 1) MAMBO_T(4, 2, 4, 1) MAMBO_T(4, 1, 8, 1) MAMBO_T(4, 1, 4, 1)
#undef MAMBO_T
    return mambo_fail(MAMBO_ERR_VALUE, "tiled kernel: no build for tile_m=%d, tile_n=%d, waves=%d", 16 * mt,
                      16 * nt * waves / ks, waves);
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Waves the default configuration aims for: about two rounds of 4 resident waves per
// SIMD (4 SIMDs x 256 CUs).
constexpr int64_t kTargetWaves = 8192;
// Below this many waves the default config splits K.
constexpr int64_t kMinWaves = 512;
// Activations are staged in LDS when the workgroup's rows take at most this much.
#ifndef MAMBO_MAX_LDS_ACT_KB
#define MAMBO_MAX_LDS_ACT_KB 40
#endif
constexpr int kMaxLdsAct = MAMBO_MAX_LDS_ACT_KB * 1024;
// Compute units of an MI355X (the tiled default sizes its grid to at least one
// workgroup per CU).
constexpr int64_t kCUs = 256;
// Workgroups the stream kernel's default aims for when it has many tiles.
constexpr int64_t kStreamWgs = 512;
// Most workgroups of a stream launch that quantizes its activations itself.
#ifndef MAMBO_FUSED_WGS
#define MAMBO_FUSED_WGS 1024
#endif
constexpr int64_t kFusedWgs = MAMBO_FUSED_WGS;
// Token count from which the default configuration uses the tiled kernel.
constexpr int64_t kTiledMinM = 64;
// Dynamic LDS per workgroup (the static codebook tables add 2.3 KiB).
#ifndef MAMBO_MAX_DYN_LDS_KB
#define MAMBO_MAX_DYN_LDS_KB 150
#endif
constexpr int kMaxDynLds = MAMBO_MAX_DYN_LDS_KB * 1024;
// LDS per CU on gfx950.
constexpr int kLdsPerCU = 160 * 1024;
// Dynamic LDS a stream-kernel workgroup may take beside its static codebook of 2^lg copies.
int stream_max_dyn_lds(int lg) { return kLdsPerCU - stream_lut_bytes(lg) - 1024; }

// Codebook copies (log2) of a stream launch with `rows` tokens per workgroup over
// `blocks` K blocks (graph-timed sweeps, one box): one copy for one token on K >= 8192
// (70B M=1: 4 copies -0.2%, 16 copies -5%: the LDS they take costs resident
// workgroups), 16 for 3-4 tokens on K >= 8192 (70B M=3 +4.7%, M=4 +8%), else 4 (70B M=2
// +2.1%, 8B M=1 +1.0%, M=4 +2.2%). Several 4-token sub-tiles (M > 4) keep one copy (4
// copies for 5-8 tokens on K = 4096: 8B M=8 sweep -3%).
int stream_copies_lg(int64_t rows, int64_t blocks)
{
    if (rows > 4)
        return 0;
    if (blocks >= 32)
        return rows == 1 ? 0 : rows >= 3 ? 4 : 2;
    return 2;
}

// Whether the stream kernel stages its chunk's activations in LDS (`lds_bytes`: the
// workgroup's whole dynamic LDS with them): when they take at most kMaxLdsAct, or when
// the LDS (with the static codebook) still leaves room for 16 waves per CU (one 16-wave
// workgroup, two 8-wave ones).
// Beyond that they are read from L2 in the weight ring.
bool stream_stages_act(int64_t act_bytes, int lds_bytes, int waves, int lg)
{
    if (lds_bytes > stream_max_dyn_lds(lg))
        return false;
    return act_bytes <= kMaxLdsAct || (int64_t)(lds_bytes + stream_lut_bytes(lg)) * 16 <= (int64_t)kLdsPerCU * waves;
}

bool valid_waves(int w)
{
    for (int v : kStreamWaves)
        if (v == w)
            return true;
    return false;
}

} // namespace

namespace {

// Default configuration of `kernel` (MAMBO_GEMM_AUTO: the family chosen by M) for the shape.
mambo_gemm_config family_default(int kernel, int64_t m, int64_t n, int64_t blocks)
{
    mambo_gemm_config c = {};
    // 17-32 tokens: the tiled kernel's 32-token tiles, four waves of 16 weight rows sharing
    // each activation block through LDS, K split until the grid holds about 512
    // workgroups (at most 4 splits of at least 8 blocks). Measured in the replayed sweeps
    // ahead of the dense kernel on all four 70B launches (2-9%) and the 8B gate/up (10%),
    // within 1% behind it on the 8B o and down launches.
    if (kernel == MAMBO_GEMM_AUTO && m > 16 && m <= 32) {
        const int64_t wgs = cdiv(cdiv(n, kTileRows), 4);
        const int64_t split = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(cdiv(512, wgs), 4), blocks / 8));
        if (wgs * split >= kCUs / 2) {
            c.kernel = MAMBO_GEMM_TILED;
            c.tile_m = 32;
            c.tile_n = 64;
            c.waves = 4;
            c.split_k = (int32_t)split;
            return c;
        }
    }
    // Block-diagonal activations cost nothing extra while one MFMA covers every token
    // (M <= 4); beyond that the dense kernel does 4 MFMAs per block for 16 tokens where
    // the block-diagonal one needs 2 per 4 tokens and an activation sub-tile each; the
    // tiled kernel from 64 tokens.
    c.kernel = kernel != MAMBO_GEMM_AUTO ? kernel
               : m <= 4                  ? MAMBO_GEMM_STREAM
               : m < kTiledMinM          ? MAMBO_GEMM_DENSE
                                         : MAMBO_GEMM_TILED;
    if (c.kernel == MAMBO_GEMM_TILED) {
        // 256 tokens x 256 weight rows x 16 waves (one workgroup per CU, half-K form) when
        // every round of its grid fills at least 7/8 of the CUs (measured on gfx950: 6-17% ahead of
        // 128 x 128 x 8 on the 8B/70B gate/up and down projections at 512-8192 tokens,
        // behind it on grids of 192 workgroups); else 128 tokens x 128 weight rows x 8
        // waves when that gives every CU a workgroup (the fastest of the 8-wave tiles or
        // within 3% of it, ahead of 256 x 128 x 8 by up to 16% where that grid ends in a
        // partial round), then 64 x 128 x 8; when even that leaves CUs idle, K is split
        // (at least 8 blocks per split) until the grid covers the chip twice.
        // On long K (at least 48 blocks: the down projections) the 128-token tile stays
        // and K is split (at least 16 blocks per split) until the grid covers the chip
        // twice (measured: 8192 x 28672 at 256 and 512 tokens, 4096 x 14336 at 512,
        // 20-30% faster than 64 x 128 tiles).
        const int64_t rt = cdiv(n, kTileRows);
        c.split_k = 1;
        c.waves = 8;
        c.tile_n = 128;
        int64_t wgs;
        // (the 128-token tile only where its token padding is within 1/8 of the 64-token
        // tile's: never for M < 128)
        const bool fits128 = m >= 128 && cdiv(m, 128) * 128 * 8 <= cdiv(m, 64) * 64 * 9;
        const bool fits256 = m >= 256 && cdiv(m, 256) * 256 * 8 <= cdiv(m, 128) * 128 * 9;
        const bool long_k = blocks >= 48;
        // (one workgroup per CU: rounds must be nearly full - 320 workgroups run as two
        // rounds, and 128 x 128 x 8 was 18% faster there)
        const int64_t w256 = cdiv(rt, 16) * cdiv(m, 256), w128 = cdiv(rt, 8) * cdiv(m, 256);
        const auto rounds_full = [](int64_t w) { return w >= kCUs * 7 / 8 && w * 8 >= cdiv(w, kCUs) * kCUs * 7; };
        // Where both 256-token tiles fill their rounds, the 256 x 128 x 8 form takes over
        // when its rounds are at least 8% fuller (the 256 x 256 tile is ~3.5% faster at
        // equal fill: 8B gate/up at 1536 tokens, 672 against 1344 workgroups; at 2048
        // tokens 896 workgroups fill 3.5 rounds against 1792 filling 7, and the 128-row
        // form is ~3% faster there, the 8B sweep +1.7%).
        const bool prefer128 = rounds_full(w128) &&
                               w128 * cdiv(w256, kCUs) * 100 >= w256 * cdiv(w128, kCUs) * 108;
        if (fits256 && rounds_full(w256) && !prefer128) {
            wgs = w256;
            c.tile_m = 256;
            c.tile_n = 256;
            c.waves = 16;
        } else if (fits256 && rounds_full(w128)) {
            // the 256 x 128 x 8 prefill form where the 256-row tile leaves CUs idle but
            // the 128-row one fills whole rounds (8B o and down projections at 2048 tokens:
            // 4-10% ahead of 128 x 128 x 8)
            wgs = w128;
            c.tile_m = 256;
        } else if (fits256 && long_k && w128 < kCUs && cdiv(kCUs, w128) <= blocks / 16 &&
                   rounds_full(w128 * cdiv(kCUs, w128))) {
            // long K with too few 256 x 128 items for a round: the prefill form with a K
            // split that fills one round (at least 16 blocks per split). Against the
            // 128-token tile's wider split, whole sweeps: 70B M=256 +1.2-1.5%, 8B M=1024
            // +0.4-0.9%; where the split cannot fill a round (8B down at 512 and 768
            // tokens: capped at 3 splits, or 1.125 rounds) it lost 1-5%, so it stays off
            wgs = w128;
            c.tile_m = 256;
            c.split_k = (int32_t)cdiv(kCUs, w128);
        } else if (fits128 && ((wgs = cdiv(rt, 8) * cdiv(m, 128)) >= kCUs || long_k)) {
            c.tile_m = 128;
            if (long_k && wgs < 2 * kCUs)
                c.split_k = (int32_t)std::max<int64_t>(1, std::min<int64_t>(cdiv(2 * kCUs, wgs), blocks / 16));
        } else {
            c.tile_m = 64;
            wgs = cdiv(rt, 8) * cdiv(m, 64);
            if (wgs < kCUs)
                c.split_k = (int32_t)std::max<int64_t>(1, std::min<int64_t>(cdiv(2 * kCUs, wgs), blocks / 8));
        }
        // Few weight rows (k/v projections) leave even the split grid small: up to 255
        // tokens the dense kernel's 16-token chunks are faster there (measured).
        if (kernel == MAMBO_GEMM_AUTO && m < 256 && wgs * c.split_k < kCUs / 2)
            return family_default(MAMBO_GEMM_DENSE, m, n, blocks);
        return c;
    }
    int64_t units = cdiv(n, kTileRows) * cdiv(m, 16); // workgroups before any K split
    // Waves per workgroup (block-diagonal kernel, measured on gfx950 at M = 1): 8 when that
    // keeps at least 4 K blocks per wave or the grid is small; 4 when 8 would leave large
    // grids with short waves; 16 for tiny grids (at most 2K waves) at M <= 4 (wider
    // sub-tiles spill at 1024 threads). The count must divide the K blocks evenly.
    // K is split only when even that leaves the chip mostly idle: a split costs a zero
    // fill and atomics, which lose to wider workgroups down to ~1K waves.
    int waves = 1;
    for (int w : {2, 4})
        if (blocks % w == 0 && blocks / w >= 2)
            waves = w;
    if (blocks % 8 == 0 && blocks / 8 >= 2 && (blocks / 8 >= 4 || units * 4 < 4096))
        waves = 8;
    if (m <= 4 && units * 16 <= kTargetWaves / 4 && blocks % 16 == 0 && blocks / 16 >= 2)
        waves = 16;
    if (c.kernel == MAMBO_GEMM_DENSE) {
        // Dense: 4 waves; above 16 tokens, 32 tokens per workgroup (each decoded tile-block
        // serves two 16-token chunks); and as many weight tiles per workgroup (sharing each
        // activation fragment) as still leave a workgroup per CU at 16 tokens, or 5/8 of
        // one at 32 (measured on gfx950: M = 8..16, and M = 24..48 on the 70B shapes).
        waves = 1;
        for (int w : {2, 4})
            if (blocks % w == 0 && blocks / w >= 2)
                waves = w;
        const int mc = m > 16 && waves >= 2 ? 2 : 1;
        c.tile_m = 16 * mc;
        const int64_t rt = cdiv(n, kTileRows), mchunks = cdiv(m, 16 * mc);
        const int64_t min_wgs = mc == 2 ? kCUs * 5 / 8 : kCUs;
        int nt = 1;
        for (int t : {2, 4})
            if (cdiv(rt, t) * mchunks >= min_wgs)
                nt = t;
        c.tile_n = kTileRows * nt;
        units = cdiv(rt, nt) * mchunks;
    }
    if (c.kernel == MAMBO_GEMM_STREAM) {
        // Runs of tiles per workgroup: about two workgroups per CU (512) walking their
        // tiles back to back beat one short-lived workgroup per tile once there are
        // several tiles per CU (measured on gfx950 at M = 1 and 4: 7 tiles per workgroup
        // for 3584 tiles, 4 for 1792, 1 for 512-640).
        c.tile_n = (int32_t)(kTileRows * std::max<int64_t>(1, (units + kStreamWgs / 2) / kStreamWgs));
        // Activations past kMaxLdsAct (M = 2..4 on K = 14K-28K): one 16-wave workgroup per
        // CU stages them once for all its waves (measured on the 70B down projection
        // 8192 x 28672: 21.3 / 22.4 / 24.1 us at M = 2 / 3 / 4 against 26-28 us with them
        // read from L2 in the ring).
        const int64_t act = std::min<int64_t>(16, m) * blocks * 256 * 33 / 32;
        if (act > kMaxLdsAct && blocks >= 32 &&
            act + 8192 <= stream_max_dyn_lds(stream_copies_lg(std::min<int64_t>(16, m), blocks))) {
            waves = 16;
            c.tile_n = (int32_t)(kTileRows * std::max<int64_t>(1, (units + kCUs / 2) / kCUs));
        }
    }
    int64_t split = 1;
    if (units * waves < (c.kernel == MAMBO_GEMM_DENSE ? kMinWaves / 4 : kMinWaves)) {
        const int64_t per_split_waves = units * waves;
        split = std::min<int64_t>(cdiv(kMinWaves, per_split_waves), std::max<int64_t>(1, blocks / (2 * waves)));
    }
    c.waves = waves;
    c.split_k = (int32_t)std::max<int64_t>(split, 1);
    return c;
}

} // namespace

extern "C" int mambo_gemm_default_config(int64_t m, int64_t n, int64_t blocks, mambo_gemm_config *out)
{
    MAMBO_REQUIRE(out != nullptr, MAMBO_ERR_VALUE, "out must not be NULL");
    MAMBO_REQUIRE(m >= 1 && n >= 1 && blocks >= 1, MAMBO_ERR_VALUE, "shape must be positive");
    *out = family_default(MAMBO_GEMM_AUTO, m, n, blocks);
    return MAMBO_OK;
}

extern "C" int mambo_gemm_check_config(int64_t m, int64_t n, int64_t blocks, const mambo_gemm_config *cfg)
{
    MAMBO_REQUIRE(cfg != nullptr, MAMBO_ERR_VALUE, "cfg must not be NULL");
    MAMBO_REQUIRE(m >= 1 && n >= 1 && blocks >= 1, MAMBO_ERR_VALUE, "shape must be positive");
    MAMBO_REQUIRE(cfg->kernel == MAMBO_GEMM_STREAM || cfg->kernel == MAMBO_GEMM_DENSE ||
                      cfg->kernel == MAMBO_GEMM_TILED,
                  MAMBO_ERR_VALUE, "unsupported kernel family %d", cfg->kernel);
    if (cfg->kernel == MAMBO_GEMM_TILED && (cfg->tile_m == 16 || cfg->tile_m == 32)) {
        if (cfg->tile_m == 16)
            MAMBO_REQUIRE((cfg->waves == 4 && (cfg->tile_n == 64 || cfg->tile_n == 128 || cfg->tile_n == 256)) ||
                              (cfg->waves == 8 && (cfg->tile_n == 64 || cfg->tile_n == 128)) ||
                              (cfg->waves == 16 && cfg->tile_n == 64) ||
                              ((cfg->waves == 4 || cfg->waves == 8 || cfg->waves == 16) &&
                               (cfg->tile_n == 16 || cfg->tile_n == 32)),
                          MAMBO_ERR_VALUE, "tiled: tile_m=16 is built for 4 waves of 16, 32 or 64 weight rows (tile_n=64, "
                                           "128 or 256), with 2 K groups of them for 16 or 32 rows (8 waves, tile_n=64 or "
                                           "128) or 4 K groups for 16 rows (16 waves, tile_n=64), and for K groups of 1 or "
                                           "2 waves of 16 rows (tile_n=16 or 32) in 4, 8 or 16 waves");
        else
            MAMBO_REQUIRE((cfg->waves == 4 && (cfg->tile_n == 64 || cfg->tile_n == 128)) ||
                              (cfg->waves == 8 && (cfg->tile_n == 16 || cfg->tile_n == 32 || cfg->tile_n == 64 ||
                                                   cfg->tile_n == 128)),
                          MAMBO_ERR_VALUE, "tiled: tile_m=32 is built for 4 waves of 16 or 32 weight rows (tile_n=64 "
                                           "or 128), 8 waves of 16 (tile_n=128) or K groups of 1, 2 or 4 waves of 16 "
                                           "in 8 waves (tile_n=16, 32 or 64)");
        MAMBO_REQUIRE(cfg->split_k >= 1 && cfg->split_k <= blocks && cfg->split_k <= 65535, MAMBO_ERR_VALUE,
                      "split_k must be in [1, K/256]");
        return MAMBO_OK;
    }
    if (cfg->kernel == MAMBO_GEMM_TILED) {
        MAMBO_REQUIRE(cfg->tile_m == 64 || cfg->tile_m == 128 || cfg->tile_m == 256, MAMBO_ERR_VALUE,
                      "tiled: tile_m must be 16, 32, 64, 128 or 256");
        MAMBO_REQUIRE(cfg->waves == 4 || cfg->waves == 8 || (cfg->waves == 16 && cfg->tile_m == 256), MAMBO_ERR_VALUE,
                      "tiled: waves must be 4 or 8 (16 only with tile_m=256)");
        MAMBO_REQUIRE(cfg->tile_n == 16 * cfg->waves || cfg->tile_n == 32 * cfg->waves, MAMBO_ERR_VALUE,
                      "tiled: tile_n must be 16 or 32 weight rows per wave");
        MAMBO_REQUIRE(cfg->tile_m != 256 || (cfg->waves == 8 && cfg->tile_n == 128) ||
                          (cfg->waves == 16 && cfg->tile_n == 256),
                      MAMBO_ERR_VALUE,
                      "tiled: tile_m=256 is built for 8 or 16 waves of 16 weight rows (tile_n=128 or 256)");
        MAMBO_REQUIRE(cfg->split_k >= 1 && cfg->split_k <= blocks && cfg->split_k <= 65535, MAMBO_ERR_VALUE,
                      "split_k must be in [1, K/256]");
        return MAMBO_OK;
    }
    MAMBO_REQUIRE(valid_waves(cfg->waves), MAMBO_ERR_VALUE, "waves must be one of 1, 2, 4, 6, 8, 12, 16");
    if (cfg->kernel == MAMBO_GEMM_DENSE) {
        MAMBO_REQUIRE(cfg->tile_n == 0 || cfg->tile_n == 16 || cfg->tile_n == 32 || cfg->tile_n == 64,
                      MAMBO_ERR_VALUE, "dense: tile_n must be 16, 32 or 64 weight rows");
        MAMBO_REQUIRE(cfg->tile_m == 0 || cfg->tile_m == 16 || cfg->tile_m == 32, MAMBO_ERR_VALUE,
                      "dense: tile_m must be 16 or 32 tokens");
        MAMBO_REQUIRE(cfg->tile_m != 32 || cfg->waves == 2 || cfg->waves == 4 || cfg->waves == 8, MAMBO_ERR_VALUE,
                      "dense: tile_m=32 is built for 2, 4 or 8 waves");
    } else
        MAMBO_REQUIRE(cfg->tile_n >= 0 && cfg->tile_n % kTileRows == 0 && cfg->tile_n <= (1 << 20), MAMBO_ERR_VALUE,
                      "stream: tile_n must be a multiple of 16 weight rows, at most 2^20");
    MAMBO_REQUIRE(cfg->split_k >= 1 && cfg->split_k <= blocks && cfg->split_k <= 65535, MAMBO_ERR_VALUE,
                  "split_k must be in [1, K/256]");
    return MAMBO_OK;
}

// Autotuner candidates for one shape (the analogue of the search spaces built in
// iq3_s_fp8.py:416-459), led by the library default (an all-zero MAMBO_GEMM_AUTO entry):
// the stream kernel up to 16 tokens and the dense kernel up to 128 (both re-read every
// weight once per 16- or 32-token chunk, so neither is a candidate beyond), each over
// waves per workgroup x K split x weight rows (and, dense above 16 tokens, tokens) per
// workgroup; for 5..64 tokens the tiled kernel's 16-token tiles (32-token ones from 17)
// and from 32 its larger tile shapes, x K split. Every entry but the first passes
// mambo_gemm_check_config for the shape.
extern "C" int64_t mambo_gemm_config_enumerate(int64_t m, int64_t n, int64_t blocks, mambo_gemm_config *out,
                                               int64_t capacity)
{
    MAMBO_REQUIRE(m >= 1 && n >= 1 && blocks >= 1, MAMBO_ERR_VALUE, "shape must be positive");
    MAMBO_REQUIRE(capacity >= 0 && (out != nullptr || capacity == 0), MAMBO_ERR_VALUE,
                  "out must hold capacity configurations");
    int64_t count = 0;
    auto add = [&](int32_t kernel, int32_t waves, int32_t split, int32_t tile_m, int32_t tile_n) {
        if (count < capacity) {
            mambo_gemm_config c = {};
            c.kernel = kernel;
            c.waves = waves;
            c.split_k = split;
            c.tile_m = tile_m;
            c.tile_n = tile_n;
            out[count] = c;
        }
        ++count;
    };
    add(MAMBO_GEMM_AUTO, 0, 0, 0, 0);
    const int64_t u = std::min<int64_t>(4, cdiv(m, 4)); // 4-token sub-tiles of the stream kernel
    static const int32_t kWaves[] = {1, 2, 4, 6, 8, 12, 16};
    static const int32_t kSplits[] = {1, 2, 4, 8};
    for (const int32_t kernel : {MAMBO_GEMM_STREAM, MAMBO_GEMM_DENSE}) {
        if (m > (kernel == MAMBO_GEMM_STREAM ? 16 : 128))
            continue;
        for (const int32_t waves : kWaves) {
            if (waves > blocks || (kernel == MAMBO_GEMM_STREAM && waves * u > 32))
                continue;
            for (const int32_t split : kSplits) {
                if (split > blocks / waves)
                    continue;
                if (kernel == MAMBO_GEMM_STREAM) { // runs of 1..8 tiles per workgroup
                    for (const int32_t rows : {16, 32, 64, 128})
                        if (split == 1 || rows == 16)
                            add(kernel, waves, split, 0, rows);
                } else { // tiles sharing one activation fragment, tokens per workgroup
                    const bool two_chunks = m > 16 && (waves == 2 || waves == 4 || waves == 8);
                    for (const int32_t rows : {16, 32, 64})
                        for (const int32_t tokens : {16, 32})
                            if ((tokens == 16 || two_chunks) && waves * rows * tokens / 16 <= 256)
                                add(kernel, waves, split, tokens, rows);
                }
            }
        }
    }
    if (m > 4 && m <= 64) { // 16-token tiles: four waves share each activation block through LDS
        for (const int32_t rows : {16, 32, 64})
            for (const int32_t groups : {1, 2, 4}) // K groups of four waves inside the workgroup
                if ((groups == 1 || (groups == 2 && rows <= 32) || rows == 16) && groups <= blocks)
                    for (const int32_t split : {1, 2, 4})
                        if (split * groups <= blocks)
                            add(MAMBO_GEMM_TILED, 4 * groups, split, 16, rows * 4);
        // K groups of one or two waves of 16 rows (4, 8 or 16 waves)
        for (const int32_t group_waves : {1, 2})
            for (const int32_t waves : {4, 8, 16})
                for (const int32_t split : {1, 2, 4})
                    if (split * (waves / group_waves) <= blocks)
                        add(MAMBO_GEMM_TILED, waves, split, 16, 16 * group_waves);
    }
    if (m > 16 && m <= 64) // 32-token tiles (8 waves: of 16 rows, tile_n 128, or K groups, tile_n 16-64)
        for (const int32_t waves : {4, 8})
            for (const int32_t rows : {16, 32})
                if (waves == 4 || rows == 16)
                    for (const int32_t split : {1, 2, 4})
                        if (split <= blocks) {
                            add(MAMBO_GEMM_TILED, waves, split, 32, rows * waves);
                            if (waves == 8) // K groups of 4, 2 or 1 waves of 16 rows
                                for (const int32_t tn : {64, 32, 16})
                                    if (split * (8 * 16 / tn) <= blocks)
                                        add(MAMBO_GEMM_TILED, waves, split, 32, tn);
                        }
    if (m >= 32) { // tokens x weight rows per wave x waves
        for (const int32_t tile_m : {64, 128, 256})
            for (const int32_t waves : {4, 8, 16})
                for (const int32_t rows : {16, 32}) {
                    const bool built = tile_m == 256 ? rows == 16 && ((waves == 8 && m >= 128) || (waves == 16 && m >= 256))
                                                     : waves != 16;
                    if (!built)
                        continue;
                    for (const int32_t split : {1, 2, 4})
                        if (split <= blocks)
                            add(MAMBO_GEMM_TILED, waves, split, tile_m, rows * waves);
                }
    }
    return count;
}

namespace {

// run_projections with quant >= 0 launched nothing: the configuration cannot quantize
// the rows inside the GEMM.
constexpr int kNotFused = 1;

// Checks and launch closure of the two streaming families (stream, dense) for
// run_projections.
int plan_streaming(const mambo_gemm_config &c, const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs,
                   int64_t m, const GroupArgs &ga, int64_t tiles, int64_t blocks, int64_t k, int bps, int splits,
                   int atomic, int quant, hipStream_t s, std::function<int(bool)> &launch)
{
    const int64_t mchunks = cdiv(m, 16);
    MAMBO_REQUIRE(tiles <= 0x7FFFFFFF && mchunks <= 65535, MAMBO_ERR_VALUE, "shape too large for one launch");
    const int rows = (int)std::min<int64_t>(16, m); // rows of the largest M chunk
    // Stage the activations in LDS when they are small enough; otherwise read them from
    // global memory (L2) in the weight ring.
    bool lds_act = (int64_t)rows * k * 33 / 32 <= kMaxLdsAct;
    dim3 grid((unsigned)tiles, (unsigned)splits, (unsigned)mchunks);
    const int B = (int)blocks;
    if (c.kernel == MAMBO_GEMM_DENSE) {
        const int nt = c.tile_n ? c.tile_n / kTileRows : 1;
        const int mc = c.tile_m == 32 ? 2 : 1; // 16-token chunks per workgroup
        const int drows = (int)std::min<int64_t>(16 * mc, m);
        // workgroups per projection (NT tiles each); tile_begin counts workgroups
        GroupArgs gd = ga;
        int64_t wgs = 0;
        for (int g = 0; g < ga.count; ++g) {
            gd.tile_begin[g] = wgs;
            wgs += cdiv(cdiv(ga.n[g], kTileRows), nt);
        }
        grid.x = (unsigned)wgs;
        grid.z = (unsigned)cdiv(m, 16 * mc);
        lds_act = (int64_t)drows * k * 33 / 32 <= kMaxLdsAct;
        if ((uintptr_t)xs % 4 != 0 || ldxs % 4 != 0) // the staging copies move scales as dwords
            lds_act = false;
        if (lds_act && dense_lds(c.waves, nt, mc, drows, (int)k, true).total > kMaxDynLds)
            lds_act = false;
        const DenseLds L = dense_lds(c.waves, nt, mc, drows, (int)k, lds_act);
        MAMBO_REQUIRE(L.total <= kMaxDynLds, MAMBO_ERR_VALUE,
                      "configuration needs %d bytes of LDS per workgroup (waves=%d, tile_n=%d, tile_m=%d)", L.total,
                      c.waves, c.tile_n, c.tile_m);
        const int waves = c.waves;
        launch = [=](bool dry) {
            return launch_dense(dry, waves, nt, mc, lds_act, grid, L.total, s, xv, ldxv, xs, ldxs, m, gd, B, bps,
                                atomic);
        };
        return MAMBO_OK;
    } else {
        const int U = (int)std::min<int64_t>(4, cdiv(m, 4));
        const int lg = stream_copies_lg(rows, blocks);
        lds_act = stream_stages_act((int64_t)rows * k * 33 / 32,
                                    stream_lds(U, c.waves, std::min(rows, 4 * U), (int)k, true).total, c.waves, lg);
        // the staging copies move activation scales as dwords
        if (quant < 0 && ((uintptr_t)xs % 4 != 0 || ldxs % 4 != 0))
            lds_act = false;
        const StreamLds L = stream_lds(U, c.waves, std::min(rows, 4 * U), (int)k, lds_act);
        MAMBO_REQUIRE(L.total <= stream_max_dyn_lds(lg), MAMBO_ERR_VALUE,
                      "configuration needs %d bytes of LDS per workgroup (waves=%d, M=%lld); use fewer waves", L.total,
                      c.waves, (long long)m);
        int64_t runs = c.tile_n ? c.tile_n / kTileRows : 1;
        // quantizing inside the GEMM repeats the rows' quantization in every workgroup:
        // longer runs keep the workgroup count (and that repeated work) bounded
        if (quant >= 0)
            runs = std::max<int64_t>(runs, cdiv(tiles, kFusedWgs));
        const int tpw = (int)std::min<int64_t>(runs, tiles);
        StreamLaunch sl = {grid, (size_t)L.total, tiles, tpw, B, bps, atomic, lg};
        sl.grid.x = (unsigned)cdiv(tiles, tpw);
        const int waves = c.waves;
        launch = [=](bool dry) {
            switch (U) {
            case 1: return launch_stream_u<1>(dry, waves, lds_act, quant, sl, s, xv, ldxv, xs, ldxs, m, ga);
            case 2: return launch_stream_u<2>(dry, waves, lds_act, -1, sl, s, xv, ldxv, xs, ldxs, m, ga);
            case 3: return launch_stream_u<3>(dry, waves, lds_act, -1, sl, s, xv, ldxv, xs, ldxs, m, ga);
            default: return launch_stream_u<4>(dry, waves, lds_act, -1, sl, s, xv, ldxv, xs, ldxs, m, ga);
            }
        };
        return MAMBO_OK;
    }
}


// quant: -1 when xv/xs are MXFP8 activations; else xv holds unquantized rows of dtype
// quant (ldxv in elements, xs unused) for the stream kernel to quantize itself, and the
// call returns kNotFused, launching nothing, when the configuration cannot do that.
int run_projections(const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t m,
                    const mambo_projection *proj, int count, int64_t blocks, const mambo_gemm_config *cfg,
                    hipStream_t s, int quant = -1)
{
    MAMBO_REQUIRE(xv && (xs || quant >= 0) && proj, MAMBO_ERR_VALUE, "null pointer");
    MAMBO_REQUIRE(count >= 1 && count <= kMaxGroup, MAMBO_ERR_VALUE, "count must be in [1, %d] (got %d)", kMaxGroup,
                  count);
    MAMBO_REQUIRE(m >= 1 && blocks >= 1, MAMBO_ERR_VALUE, "shape must be positive (M=%lld B=%lld)", (long long)m,
                  (long long)blocks);
    MAMBO_REQUIRE(blocks <= (1 << 20), MAMBO_ERR_VALUE, "K too large");
    const int64_t k = blocks * 256;
    MAMBO_REQUIRE(ldxv >= k && (quant >= 0 || ldxs >= k / 32), MAMBO_ERR_VALUE,
                  "activation row strides must cover the row");
    MAMBO_REQUIRE(ldxv < ((int64_t)1 << 27) && (quant >= 0 || ldxs < ((int64_t)1 << 27)), MAMBO_ERR_VALUE,
                  "activation row stride too large");
    if (quant < 0)
        MAMBO_REQUIRE((uintptr_t)xv % 16 == 0 && ldxv % 16 == 0, MAMBO_ERR_VALUE,
                      "x_values base and row stride must be 16-byte aligned");
    GroupArgs ga = {};
    ga.count = count;
    int64_t tiles = 0, n_total = 0;
    for (int g = 0; g < count; ++g) {
        const mambo_projection &p = proj[g];
        MAMBO_REQUIRE(p.packed && p.out, MAMBO_ERR_VALUE, "projection %d: null pointer", g);
        MAMBO_REQUIRE(p.n >= 1, MAMBO_ERR_VALUE, "projection %d: n must be positive (N=%lld)", g, (long long)p.n);
        MAMBO_REQUIRE(p.ldo >= p.n, MAMBO_ERR_VALUE, "projection %d: output row stride must cover the row", g);
        MAMBO_REQUIRE((uintptr_t)p.packed % 16 == 0, MAMBO_ERR_VALUE, "projection %d: packed weight must be 16-byte aligned", g);
        ga.packed[g] = p.packed;
        ga.out[g] = p.out;
        ga.n[g] = p.n;
        ga.ldo[g] = p.ldo;
        ga.tile_begin[g] = tiles;
        tiles += cdiv(p.n, kTileRows);
        n_total += p.n;
    }
    // Library default of the requested kernel family (or of the family chosen by M),
    // overlaid with the non-zero fields of cfg.
    MAMBO_REQUIRE(cfg == nullptr || (cfg->kernel >= MAMBO_GEMM_AUTO && cfg->kernel <= MAMBO_GEMM_DENSE),
                  MAMBO_ERR_VALUE, "unsupported kernel family %d", cfg ? cfg->kernel : 0);
    mambo_gemm_config c = family_default(cfg ? cfg->kernel : MAMBO_GEMM_AUTO, m, n_total, blocks);
    int rc = MAMBO_OK;
    if (cfg != nullptr) {
        if (cfg->waves)
            c.waves = cfg->waves;
        if (cfg->split_k)
            c.split_k = cfg->split_k;
        if (cfg->tile_m)
            c.tile_m = cfg->tile_m;
        if (cfg->tile_n)
            c.tile_n = cfg->tile_n;
        rc = mambo_gemm_check_config(m, n_total, blocks, &c);
        if (rc)
            return rc;
    }
    if (quant >= 0) { // in-kernel quantization: stream kernel, one sub-tile, rows staged in LDS
        const int64_t esz = quant == MAMBO_DTYPE_BF16 ? 2 : 4;
        const int qrows = (int)std::min<int64_t>(4, m);
        const int qlds = stream_lds(1, c.waves, qrows, (int)k, true).total;
        const int qlg = stream_copies_lg(qrows, blocks);
        if (c.kernel != MAMBO_GEMM_STREAM || m > 4 || (uintptr_t)xv % 16 != 0 || (ldxv * esz) % 16 != 0 ||
            !stream_stages_act((int64_t)qrows * k * 33 / 32, qlds, c.waves, qlg) || qlds > stream_max_dyn_lds(qlg))
            return kNotFused;
    }
    const int bps = (int)cdiv(blocks, c.split_k);
    const int splits = (int)cdiv(blocks, bps);
    const int atomic = splits > 1;
    if (atomic)
        MAMBO_REQUIRE(m <= 65535, MAMBO_ERR_VALUE, "M too large for split-K");
    // The launch of the chosen family: dry = true checks that it is built, launching
    // nothing. Every check runs before the K split's zero fill is queued, so a rejected
    // call leaves the outputs and the stream untouched.
    std::function<int(bool)> launch;
    const char *what = "iq3s_fp8_matmul";
    if (c.kernel == MAMBO_GEMM_TILED) {
        const int ks = tiled_groups(c), tw = c.waves / ks;
        const int mt = c.tile_m / 16, nt = c.tile_n / (16 * tw);
        MAMBO_REQUIRE((uintptr_t)xs % 8 == 0 && ldxs % 8 == 0, MAMBO_ERR_VALUE,
                      "tiled: x_scales base and row stride must be 8-byte aligned");
        // the staging copies address a token tile with 32-bit offsets
        MAMBO_REQUIRE((int64_t)c.tile_m * ldxv < ((int64_t)1 << 32) && (int64_t)c.tile_m * ldxs < ((int64_t)1 << 32),
                      MAMBO_ERR_VALUE, "tiled: activation row stride too large for tile_m=%d", c.tile_m);
        // workgroups per projection; tile_begin counts workgroups for this kernel
        GroupArgs gt = ga;
        int64_t wgs = 0;
        for (int g = 0; g < count; ++g) {
            gt.tile_begin[g] = wgs;
            wgs += cdiv(cdiv(ga.n[g], kTileRows), (int64_t)nt * tw);
        }
        const int64_t mtiles = cdiv(m, c.tile_m);
        MAMBO_REQUIRE(wgs <= 0x7FFFFFFF && mtiles <= 65535, MAMBO_ERR_VALUE, "shape too large for one launch");
        const dim3 grid((unsigned)wgs, (unsigned)mtiles, (unsigned)splits);
        launch = [=](bool dry) {
            return launch_tiled(dry, mt, nt, c.waves, ks, grid, s, xv, ldxv, xs, ldxs, m, gt, (int)blocks, bps,
                                atomic);
        };
        what = "iq3s_fp8_matmul (tiled)";
    } else {
        rc = plan_streaming(c, xv, ldxv, xs, ldxs, m, ga, tiles, blocks, k, bps, splits, atomic, quant, s, launch);
        if (rc)
            return rc;
    }
    rc = launch(true);
    if (rc)
        return rc;
    if (atomic) {
        int64_t n_max = 0;
        for (int g = 0; g < count; ++g)
            n_max = std::max(n_max, ga.n[g]);
        const int64_t chunks = m * cdiv(n_max, 4); // 4-float chunks of the widest projection
        MAMBO_REQUIRE(chunks <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "output too large for one split-K launch");
        dim3 zg((unsigned)std::min<int64_t>(cdiv(chunks, 256), 1024), (unsigned)count);
        MAMBO_LAUNCH(zero_rows_kernel, zg, dim3(256), 0, s, ga, (int)m);
        rc = mambo_check_launch("zero_rows");
        if (rc)
            return rc;
    }
    rc = launch(false);
    if (rc)
        return rc;
    return mambo_check_launch(what);
}

} // namespace

extern "C" int mambo_iq3s_fp8_matmul(const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs, int64_t m,
                                     const uint8_t *packed, int64_t n, int64_t blocks, float *out, int64_t ldo,
                                     const mambo_gemm_config *cfg, mambo_stream_t stream)
{
    MAMBO_REQUIRE(packed && out, MAMBO_ERR_VALUE, "null pointer");
    MAMBO_REQUIRE(n >= 1, MAMBO_ERR_VALUE, "shape must be positive (N=%lld)", (long long)n);
    MAMBO_REQUIRE(ldo >= n, MAMBO_ERR_VALUE, "row strides must cover the row");
    const mambo_projection p = {packed, n, out, ldo};
    return run_projections(xv, ldxv, xs, ldxs, m, &p, 1, blocks, cfg, (hipStream_t)stream);
}

extern "C" int mambo_iq3s_fp8_matmul_grouped(const uint8_t *xv, int64_t ldxv, const uint8_t *xs, int64_t ldxs,
                                             int64_t m, const mambo_projection *proj, int count, int64_t blocks,
                                             const mambo_gemm_config *cfg, mambo_stream_t stream)
{
    return run_projections(xv, ldxv, xs, ldxs, m, proj, count, blocks, cfg, (hipStream_t)stream);
}

extern "C" int mambo_iq3s_matmul_quantize_grouped(const void *x, int x_dtype, int64_t ldx, int64_t m,
                                                  const mambo_projection *proj, int count, int64_t blocks,
                                                  const mambo_gemm_config *cfg, uint8_t *xv, int64_t ldxv,
                                                  uint8_t *xs, int64_t ldxs, mambo_stream_t stream)
{
    MAMBO_REQUIRE(x_dtype == MAMBO_DTYPE_F32 || x_dtype == MAMBO_DTYPE_BF16, MAMBO_ERR_VALUE,
                  "activation dtype must be float32 or bfloat16");
    MAMBO_REQUIRE(x && xv && xs, MAMBO_ERR_VALUE, "null pointer");
    MAMBO_REQUIRE(m >= 1 && blocks >= 1 && blocks <= (1 << 20), MAMBO_ERR_VALUE, "shape must be positive");
    const hipStream_t s = (hipStream_t)stream;
    const int rc = run_projections(reinterpret_cast<const uint8_t *>(x), ldx, nullptr, 0, m, proj, count, blocks, cfg,
                                   s, x_dtype);
    if (rc != kNotFused)
        return rc;
    const int qrc = mambo_quantize_mxfp8(x, x_dtype, m, blocks * 256, ldx, xv, ldxv, xs, ldxs, stream);
    if (qrc)
        return qrc;
    return run_projections(xv, ldxv, xs, ldxs, m, proj, count, blocks, cfg, s);
}

// ---------------------------------------------------------------- no-allocation variant
// Staging array of mambo_iq3s_matmul_quantize_grouped_noalloc: the MXFP8 rows of a call
// whose rows are not quantized inside the GEMM (values [m, K] at offset 0, scales
// [m, K/32] at the next 256-byte boundary). One copy per GPU, held until the process
// ends. Host code never passes the array's name: it is a host-side stand-in, and each
// GPU holds its own copy at its own address, which hipGetSymbolAddress gives per device.
namespace {
static __device__ __align__(256) uint8_t scratch[MAMBO_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device (with that device
// current) and kept.
int scratch_address(uint8_t **out)
{
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess)
        return mambo_fail(MAMBO_ERR_RUNTIME, "hipGetDevice: %s", hipGetErrorString(err));
    MAMBO_REQUIRE(dev >= 0 && dev < kMaxDevices, MAMBO_ERR_UNSUPPORTED, "device %d beyond the library's %d", dev,
                  kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void *ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || ptr == nullptr)
            return mambo_fail(MAMBO_ERR_RUNTIME, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                              hipGetErrorString(err));
        g_scratch_ptr[dev] = static_cast<uint8_t *>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return MAMBO_OK;
}
} // namespace

extern "C" int mambo_iq3s_matmul_quantize_grouped_noalloc(const void *x, int x_dtype, int64_t ldx, int64_t m,
                                                          const mambo_projection *proj, int count, int64_t blocks,
                                                          const mambo_gemm_config *cfg, mambo_stream_t stream)
{
    MAMBO_REQUIRE(x_dtype == MAMBO_DTYPE_F32 || x_dtype == MAMBO_DTYPE_BF16, MAMBO_ERR_VALUE,
                  "activation dtype must be float32 or bfloat16");
    MAMBO_REQUIRE(x, MAMBO_ERR_VALUE, "null pointer");
    MAMBO_REQUIRE(m >= 1 && blocks >= 1 && blocks <= (1 << 20), MAMBO_ERR_VALUE, "shape must be positive");
    const int64_t k = blocks * 256;
    const int64_t xs_off = (m * k + 255) / 256 * 256;
    MAMBO_REQUIRE(m <= MAMBO_NOALLOC_SCRATCH_BYTES / k && xs_off + m * (k / 32) <= MAMBO_NOALLOC_SCRATCH_BYTES,
                  MAMBO_ERR_VALUE,
                  "noalloc: %lld rows of K=%lld need %lld bytes of MXFP8 staging, beyond the library's %d",
                  (long long)m, (long long)k, (long long)(xs_off + m * (k / 32)), MAMBO_NOALLOC_SCRATCH_BYTES);
    uint8_t *ptr = nullptr;
    int rc = scratch_address(&ptr);
    if (rc)
        return rc;
    const hipStream_t s = (hipStream_t)stream;
    rc = run_projections(reinterpret_cast<const uint8_t *>(x), ldx, nullptr, 0, m, proj, count, blocks, cfg, s,
                         x_dtype);
    if (rc != kNotFused)
        return rc;
    rc = mambo_quantize_mxfp8(x, x_dtype, m, k, ldx, ptr, k, ptr + xs_off, k / 32, stream);
    if (rc)
        return rc;
    return run_projections(ptr, k, ptr + xs_off, k / 32, m, proj, count, blocks, cfg, s);
}
