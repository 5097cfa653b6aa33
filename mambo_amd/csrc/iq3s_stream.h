// Device helpers of the weight-streaming projection kernels (gemm_stream_kernel in
// iq3s_gemm.hip, gemm_chain_kernel in iq3s_chain.hip) and the tables, operand layouts and
// addressing the other GEMM families share: the per-lane tile-block loads, the codebook
// decode into MFMA operands, the block-diagonal activation operand, the grouped-launch
// arguments and the tile-end reduction. The design is described at the top of iq3s_gemm.hip.
#pragma once
#include <functional>

#include "mambo_common.h"

namespace {


__constant__ GridTables c_grid = kGridTables;

// Operands of lanes outside the block-diagonal activation tile: 64 zero bytes and two
// unit E8M0 scales (2^0).
// Kept in the global address space (not constant) so the activation pointers stay
// global and the loads are global_load, not flat_load.
__device__ __align__(16) uint8_t g_zero_chunk[64] = {};
__device__ __align__(4) uint8_t g_unit_scales[2] = {127, 127};
__constant__ SplitTables c_split = kSplitTables;

// The stream kernel's codebook in LDS holds 2^kLg copies of every E4M3 grid word: word
// idx of copy c at dword (idx << kLg) + c, and lane l reads copy l mod 2^kLg. With 16
// copies copy c lies in the banks c + 16j, so the 64 random lookups of an instruction
// collide only within the 4 lanes that share a copy, where with one copy they all hash
// into the same banks (one copy at M = 1 on 57344 x 8192: bank conflicts held the LDS
// ~57% of its active time, SQ_LDS_BANK_CONFLICT against SQ_LDS_IDX_ACTIVE). More copies
// cost LDS and so resident workgroups: stream_copies_lg picks the count per launch.
// Each image is copied into LDS as it lies here (direct copies: 16-byte, 4-byte for one
// copy).
template <int kLg>
struct RepGrid {
    uint32_t w[512 << kLg];
};
template <int kLg>
constexpr RepGrid<kLg> make_rep_grid()
{
    RepGrid<kLg> r{};
    for (int i = 0; i < (512 << kLg); ++i)
        r.w[i] = kGridTables.fp8[i >> kLg];
    return r;
}
__device__ __align__(16) const RepGrid<0> g_rep_grid0 = make_rep_grid<0>();
__device__ __align__(16) const RepGrid<2> g_rep_grid2 = make_rep_grid<2>();
__device__ __align__(16) const RepGrid<4> g_rep_grid4 = make_rep_grid<4>();

template <int kLg>
__device__ __forceinline__ const uint32_t *rep_grid()
{
    static_assert(kLg == 0 || kLg == 2 || kLg == 4, "built for 1, 4 and 16 codebook copies");
    if constexpr (kLg == 0)
        return g_rep_grid0.w;
    else if constexpr (kLg == 2)
        return g_rep_grid2.w;
    else
        return g_rep_grid4.w;
}

// LDS bytes of the codebook with 2^lg copies.
__host__ __device__ constexpr int stream_lut_bytes(int lg) { return 2048 << lg; }

// Super-blocks in flight per wave (register ring depth).
#ifndef MAMBO_STREAM_DEPTH
#define MAMBO_STREAM_DEPTH 2
#endif
constexpr int kDepth = MAMBO_STREAM_DEPTH;

// Scheduler fences that keep each step's prefetch loads ahead of its decode (without
// them the compiler sinks the loads toward their use and the ring stops overlapping).
#ifndef MAMBO_SCHED_FENCE
#define MAMBO_SCHED_FENCE 1
#endif



struct WTile {
    uint4 ia;     // idx stream bits 0..127
    uint16_t ib;  // idx stream bits 128..143
    uint2 sg;     // transposed sign words of the halves h = 0, 1
    uint8_t sc;   // scale byte q of row col: nibbles of groups 2q, 2q+1
    uint16_t dh;  // fp16 d of row col
};

// Buffer resource over the 4 GiB that start at `base` (raw, unswizzled): loads through
// it take a scalar base, a 32-bit lane offset, a scalar step offset and an immediate
// field offset, with no per-lane 64-bit address arithmetic. The host keeps every offset
// below 2^32 (run_projections checks the activation strides; weight offsets are at most
// K/256 * 1760 bytes per tile).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t byte_rsrc(const void *base)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)0xFFFFFFFFu, 0x00020000);
}

// LDS destination of the direct global-to-LDS copies.
typedef __attribute__((address_space(3))) void *lds_ptr;

// One lane's share of a tile-block (load_w_rsrc): the block at byte `step` past the
// resource base, in kWLoads vector memory instructions (codes b128 + b16, signs b64,
// the scale byte b8, the row's fp16 d b16).
constexpr int kWLoads = 5;
// Cache policy of the decode kernels' weight loads: non-temporal (gfx940-family CPol NT
// bit). Each weight byte is read once per launch; marking the stream for early eviction
// keeps the codebook and the activations in L2 (70B M=1 sweep: 6.25 -> 5.90 ms on one
// box, 6.37 -> 6.26 on another). SC0 alone measured no change, SC1 1-2% slower. The
// tiled kernel re-reads each weight tile once per token tile and keeps the default
// policy (NT measured 5% slower at M=2048).
constexpr int kStreamPolicy = 2;

template <int kPolicy = kStreamPolicy>
__device__ __forceinline__ WTile load_w_rsrc(__amdgpu_buffer_rsrc_t r, uint32_t step, uint32_t lane, uint32_t col)
{
    constexpr int kWeightPolicy = kPolicy;
    WTile w;
    const auto ia = __builtin_amdgcn_raw_buffer_load_b128(r, 16u * lane + kTileIdxA, step, kWeightPolicy);
    w.ia = uint4{ia[0], ia[1], ia[2], ia[3]};
    w.ib = __builtin_amdgcn_raw_buffer_load_b16(r, 2u * lane + kTileIdxB, step, kWeightPolicy);
    const auto sg = __builtin_amdgcn_raw_buffer_load_b64(r, 8u * lane + kTileSigns, step, kWeightPolicy);
    w.sg = uint2{sg[0], sg[1]};
    w.sc = __builtin_amdgcn_raw_buffer_load_b8(r, lane + kTileScales, step, kWeightPolicy);
    w.dh = __builtin_amdgcn_raw_buffer_load_b16(r, 2u * col + kTileD, step, kWeightPolicy);
    return w;
}

// The dense operands' scale nibbles from the lane's scale byte (WTile::sc: scales[q] of
// its row, groups 2q and 2q+1): the 16 bits of groups 4qq .. 4qq+3 (qq = q >> 1), nibble
// h = group tile_group(qq, h) (operand bytes 0-15 of half h), nibble 2 + h = group
// tile_group(2 + qq, h) (bytes 16-31). Bytes 2qq and 2qq+1 are the scale bytes of lane
// groups 2qq and 2qq+1, so one row swap brings in the partner's: after
// v_permlane16_swap(x, x) the first result holds the even lane group's byte and the
// second the odd one's, in both lanes of the pair. All 64 lanes must be active.
__device__ __forceinline__ uint32_t dense_scales(uint32_t sc)
{
    const auto r = __builtin_amdgcn_permlane16_swap(sc, sc, false, false);
    return r[0] | (r[1] << 8);
}

// Byte address (idx << 2) of code I's grid word; idx = bits [9I, 9I+9) of the stream.
template <int I>
__device__ __forceinline__ uint32_t code_addr(const uint32_t (&s)[5])
{
    constexpr int p = 9 * I - 2;
    if constexpr (p < 0) {
        return (s[0] << 2) & 0x7FCu;
    } else {
        constexpr int wi = p >> 5, sh = p & 31;
        if constexpr (wi + 1 <= 4)
            return funnel_shr(s[wi + 1], s[wi], sh) & 0x7FCu;
        else
            return (s[wi] >> sh) & 0x7FCu;
    }
}

// Byte address of code I's grid word in the codebook with 2^kLg copies, copy c4 / 4:
// (idx << (kLg + 2)) + c4 (one shift or funnel shift and one and-or).
template <int I, int kLg>
__device__ __forceinline__ uint32_t rep_addr(const uint32_t (&s)[5], uint32_t c4)
{
    constexpr uint32_t kMask = 0x7FCu << kLg;
    constexpr int p = 9 * I - 2 - kLg;
    if constexpr (p < 0) {
        return ((s[0] << (-p)) & kMask) | c4;
    } else {
        constexpr int wi = p >> 5, sh = p & 31;
        if constexpr (wi + 1 <= 4)
            return (funnel_shr(s[wi + 1], s[wi], sh) & kMask) | c4;
        else
            return ((s[wi] >> sh) & kMask) | c4;
    }
}

// Signed E4M3 word of code C (0..7) of a group: grid magnitudes with the four sign
// bits of the code moved onto bits 7, 15, 23, 31 by one rotate of the transposed word.
template <int C>
__device__ __forceinline__ uint32_t signed_word(uint32_t mag, uint32_t p)
{
    const uint32_t rot = funnel_shr(p, p, (25 + C) & 31);
    return (rot & 0x80808080u) | mag;
}

// lut: the codebook with 2^kLg copies; c4: this lane's copy offset, 4 * (lane mod 2^kLg).
template <int H, int kLg, int... C>
__device__ __forceinline__ v8i decode_group(const uint32_t (&s)[5], uint32_t p, const uint8_t *lut, uint32_t c4,
                                            std::integer_sequence<int, C...>)
{
    v8i b;
    ((b[C] = (int)signed_word<C>(*reinterpret_cast<const uint32_t *>(lut + rep_addr<8 * H + C, kLg>(s, c4)), p)), ...);
    return b;
}

// Codebook reads of a tile-block in batches of kB (16 codes per lane): batch k+1's reads
// are issued before batch k's words are used (sched_barrier fences keep the order), so
// the waits before the sign operations are partial and up to 2kB reads are in flight.
// The compiler's own order pairs each read with its use, waiting for every read: 16 LDS
// round trips per step in series, which the last step of each workgroup exposes at the
// end of a launch. One copy (M = 1), batches of 4: 70B M=1 sweep +1.1%, 8B +0.9% (2: +0.9
// / +0.4%, 8: +0.8 / -0.2%, 80 VGPRs); with 4 or 16 copies (M = 2..4) no gain.
template <int kLg, int I0, int N>
__device__ __forceinline__ void fetch_codes(const uint32_t (&s)[5], const uint8_t *lut, uint32_t c4,
                                            uint32_t (&mag)[16])
{
    if constexpr (N > 0) {
        mag[I0] = *reinterpret_cast<const uint32_t *>(lut + rep_addr<I0, kLg>(s, c4));
        fetch_codes<kLg, I0 + 1, N - 1>(s, lut, c4, mag);
    }
}
template <int I0, int N>
__device__ __forceinline__ void sign_codes(const uint32_t (&mag)[16], uint32_t p0, uint32_t p1, v8i &b0, v8i &b1)
{
    if constexpr (N > 0) {
        constexpr int C = I0 % 8;
        if constexpr (I0 < 8)
            b0[C] = (int)signed_word<C>(mag[I0], p0);
        else
            b1[C] = (int)signed_word<C>(mag[I0], p1);
        sign_codes<I0 + 1, N - 1>(mag, p0, p1, b0, b1);
    }
}
// Batches K .. KEnd-1 (of 16 / kB); a caller may stop after the batches of b0 (codes 0-7)
// and continue later with the rest.
template <int kLg, int kB, int K = 0, int KEnd = 16 / kB>
__device__ __forceinline__ void decode_batched(const uint32_t (&s)[5], uint32_t p0, uint32_t p1, const uint8_t *lut,
                                               uint32_t c4, uint32_t (&mag)[16], v8i &b0, v8i &b1)
{
    static_assert(16 % kB == 0, "batches must cover the 16 codes");
    if constexpr (K == 0)
        fetch_codes<kLg, 0, kB>(s, lut, c4, mag);
    if constexpr ((K + 1) * kB < 16) {
        __builtin_amdgcn_sched_barrier(0);
        fetch_codes<kLg, (K + 1) * kB, kB>(s, lut, c4, mag);
    }
    __builtin_amdgcn_sched_barrier(0);
    sign_codes<K * kB, kB>(mag, p0, p1, b0, b1);
    if constexpr (K + 1 < KEnd)
        decode_batched<kLg, kB, K + 1, KEnd>(s, p0, p1, lut, c4, mag, b0, b1);
}

template <int U>
struct ATile {
    v8i a[U][2];
    int s[U]; // E8M0 scales of the two K halves in bytes 0 and 1 (the MFMA picks byte h)
};

// Activation operand of one lane. Data: row i = 4*g + m' of A holds activation row m'
// only in K block kb = out_block(g) (block-diagonal), so output row i, which lane group g
// holds, sums exactly weight group tile_group(kb, h) of its column: the groups of scale
// byte g, the byte that lane group g loads (post-scale by its own F, no cross-lane
// moves). Lane l holds row i = l & 15 at K [16q, 16q+16) (bytes 0-15, in K block q >> 1)
// and [64+16q, 64+16q+16) (bytes 16-31, K block 2 + (q >> 1)), q = l >> 4: its 16
// activation bytes sit in the low half when kb < 2, the high half otherwise, and only
// when kb & 1 == q >> 1. Scales: the E8M0 scale of (row i, K block kb) comes from lane
// i + 16*kb (see a_lane). Halves off the diagonal (and rows past M) point at a zero
// chunk / unit scales with a zero stride.
struct ALane {
    const uint8_t *x;    // activation bytes of this lane's non-zero half (or zero), block 0
    const uint8_t *s;    // E8M0 scale of this lane's K block, block 0
    int xstep;           // 256 or 0
    int sstep;           // 8 or 0
    bool hi;             // the non-zero half is bytes 16-31
};

// zero: 64 zero bytes (the other half of every lane reads 16 of them). kAligned: the
// scale rows are 2-byte aligned (the LDS copy), so both scale bytes come in one read.
template <int U, bool kAligned = true>
__device__ __forceinline__ void load_a(ATile<U> &at, const ALane (&al)[U], int b, const uint8_t *zero)
{
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint8_t *xp = al[u].x + b * al[u].xstep;
        const uint8_t *xl = al[u].hi ? zero : xp;
        const uint8_t *xh = al[u].hi ? xp : zero;
        const uint8_t *sp = al[u].s + b * al[u].sstep;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 lo = *reinterpret_cast<const uint4 *>(xl + 32 * h);
            const uint4 hi = *reinterpret_cast<const uint4 *>(xh + 32 * h);
            at.a[u][h] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
        // groups tile_group(kb, 0) and tile_group(kb, 1): adjacent bytes
        if constexpr (kAligned)
            at.s[u] = *reinterpret_cast<const uint16_t *>(sp);
        else
            at.s[u] = (int)sp[0] | ((int)sp[1] << 8);
    }
}

// K block whose weight groups tile_group(kb, 0..1) make up scale byte g: the bit swap
// {0, 2, 1, 3}.
__host__ __device__ constexpr int out_block(int g) { return ((g & 1) << 1) | (g >> 1); }

// The stream kernels' LDS copy of the activation rows: 16-byte chunk c of row r lies at
// chunk slot act_slot(c, r) of the row, a permutation inside each 256-byte block (c and
// slot differ in bits 2-3 only), so that the four rows one operand read reaches at the
// same K position fall in different banks instead of all in the same ones (rows lie K
// bytes apart). An involution: the slot of a chunk and the chunk of a slot are the same.
__host__ __device__ constexpr int act_slot(int c, int r) { return c ^ (4 * (r & 3)); }

// Operand pointers of lane `lane` for the block-diagonal A above: token row r of the
// chunk (r = 4u + (lane & 3)) has its activation bytes at `row` and its scales at `srow`;
// `valid` is false when r is past M. `zero` = 64 zero bytes, `unit` = two unit scales.
// kSwizzled: `row` is an LDS copy in the act_slot order. Selects only (no indexing by a
// lane-dependent value), so everything stays in registers.
template <bool kSwizzled>
__device__ __forceinline__ ALane a_lane(int lane, bool valid, const uint8_t *row, const uint8_t *srow,
                                        const uint8_t *zero, const uint8_t *unit)
{
    const int kb = out_block((lane & 15) >> 2), q = lane >> 4;
    const bool on = valid && (kb & 1) == (q >> 1);
    // chunk of K half 0; half 1 is 2 chunks on (bit 1, which act_slot leaves alone)
    const int c0 = 2 * tile_group(kb, 0) + (q & 1);
    ALane a;
    a.x = on ? row + 16 * (kSwizzled ? act_slot(c0, lane & 3) : c0) : zero;
    a.xstep = on ? 256 : 0;
    a.hi = kb >= 2;
    // Every lane of row i carries the row's own scale, also for the K blocks where the
    // row is zero (0 x any scale adds nothing, and a non-finite scale reaches only the
    // row's own output, as its own block already does). Only the four lanes q == kb
    // reading it and the rest a shared unit scale measured 5% slower at 4 tokens.
    a.s = valid ? srow + tile_group(kb, 0) : unit;
    a.sstep = valid ? 8 : 0;
    return a;
}

template <int U, int kLg>
__device__ __forceinline__ void compute_block(const WTile &w, const ATile<U> &at, const uint8_t *lut, uint32_t c4,
                                              float (&acc)[U][4], bool valid)
{
    const uint32_t s[5] = {w.ia.x, w.ia.y, w.ia.z, w.ia.w, (uint32_t)w.ib};
    const float d = half_bits_to_float((uint16_t)w.dh);
    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
    v8i b0, b1;
    v4f c0[U];
    if constexpr (kLg == 0) {
        // half 0's MFMAs go out as soon as its codes are decoded, ahead of the waits for
        // half 1's codebook reads (left to the scheduler, they waited for every read)
        uint32_t mag[16];
        decode_batched<kLg, 4, 0, 2>(s, w.sg.x, w.sg.y, lut, c4, mag, b0, b1);
#pragma unroll
        for (int u = 0; u < U; ++u)
            c0[u] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(at.a[u][0], b0, zero, 0, 0, 0, at.s[u], 0, 127);
        decode_batched<kLg, 4, 2>(s, w.sg.x, w.sg.y, lut, c4, mag, b0, b1);
    } else {
        b0 = decode_group<0, kLg>(s, w.sg.x, lut, c4, std::make_integer_sequence<int, 8>{});
        b1 = decode_group<1, kLg>(s, w.sg.y, lut, c4, std::make_integer_sequence<int, 8>{});
#pragma unroll
        for (int u = 0; u < U; ++u)
            c0[u] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(at.a[u][0], b0, zero, 0, 0, 0, at.s[u], 0, 127);
    }
    const uint32_t sc = w.sc;
    // A block past the wave's range (a duplicate of its last block) contributes nothing.
    const float f0 = valid ? d * (float)(1u + 2u * (sc & 15u)) : 0.0f;
    const float f1 = valid ? d * (float)(1u + 2u * (sc >> 4)) : 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        v4f c1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(at.a[u][1], b1, zero, 0, 0, 1, at.s[u], 0, 127);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[u][r] = __builtin_fmaf(c1[r], f1, __builtin_fmaf(c0[u][r], f0, acc[u][r]));
    }
}

// Dynamic LDS of the stream kernel (the codebook sits in static LDS, so its address is a
// compile-time constant folded into the reads): cross-wave partial sums of a tile,
// [2][W][U][4][16] f32 (double-buffered, so one barrier per tile suffices), a zero chunk
// + unit scales for lanes off the block diagonal, and - when kLdsAct - the workgroup's
// activation rows [rows][K] and scales [rows][K/32].
struct StreamLds {
    int red, zero, x, xs, total;
};

__host__ __device__ inline StreamLds stream_lds(int U, int W, int rows, int K, bool lds_act)
{
    StreamLds l;
    l.red = 0;
    l.zero = l.red + (W > 1 ? 2 * W * U * 4 * 16 * 4 : 0);
    l.x = l.zero + 80;
    l.xs = l.x + (lds_act ? rows * K : 0);
    l.total = l.xs + (lds_act ? rows * (K / 32) : 0);
    return l;
}

// Projections of one launch: they share the activations and K; their 16-row tiles are
// numbered consecutively, projection g owning tiles [tile_begin[g], tile_begin[g+1]).
constexpr int kMaxGroup = MAMBO_MAX_GROUP;
struct GroupArgs {
    const uint8_t *packed[kMaxGroup];
    float *out[kMaxGroup];
    int64_t n[kMaxGroup];
    int64_t ldo[kMaxGroup];
    int64_t tile_begin[kMaxGroup];
    int count;
};

// Tile t of a launch: its first super-block, and its projection's output, N, row stride
// and tile index within the projection. Only constant indices into the arguments, so
// everything stays in scalar registers.
struct TileRef {
    const uint8_t *w;
    float *out;
    int64_t n, ldo, lt;
};

__device__ __forceinline__ TileRef tile_ref(const GroupArgs &ga, int64_t t, int B)
{
    TileRef r = {ga.packed[0], ga.out[0], ga.n[0], ga.ldo[0], t};
#pragma unroll
    for (int g = 1; g < kMaxGroup; ++g)
        if (g < ga.count && t >= ga.tile_begin[g]) {
            r.w = ga.packed[g];
            r.out = ga.out[g];
            r.n = ga.n[g];
            r.ldo = ga.ldo[g];
            r.lt = t - ga.tile_begin[g];
        }
    r.w += r.lt * (int64_t)B * kTileBytes;
    return r;
}

// Position of a wave in its workgroup's run of (tile, step) pairs: step i of a tile is
// super-block first + i*W; `w` is a buffer resource starting at the tile's first
// super-block.
struct StreamCursor {
    int s, i;
    int64_t t;
    __amdgpu_buffer_rsrc_t w;
};

// Move to the next pair unless at the last one (the ring's tail keeps re-reading it).
__device__ __forceinline__ void advance(StreamCursor &c, int total, int steps, const GroupArgs &ga, int B)
{
    if (c.s + 1 < total) {
        ++c.s;
        if (++c.i == steps) {
            c.i = 0;
            ++c.t;
            c.w = byte_rsrc(tile_ref(ga, c.t, B).w);
        }
    }
}

// Sum of a value over the four 16-lane groups, in every lane: v + v[l^16], then + [l^32],
// by row swaps in the VALU (v_permlane16_swap / v_permlane32_swap) instead of LDS
// permutes; a + b is commutative, so every lane gets the bits of the shuffle form.
__device__ __forceinline__ float lane_group_sum(float v)
{
    const uint32_t x = __float_as_uint(v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    const float s16 = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const uint32_t y = __float_as_uint(s16);
    const auto r32 = __builtin_amdgcn_permlane32_swap(y, y, false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// Store of one output: plain, or (kCoherent) at device scope (global_store sc1, written
// through to where every XCD reads it) for outputs that a later launch of the same
// persistent kernel may read.
template <bool kCoherent>
__device__ __forceinline__ void store_out(float *o, float v)
{
    if constexpr (kCoherent)
        __hip_atomic_store(o, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *o = v;
}

// End of a tile: sum the wave's four K chunks (lane groups), then the waves' sums through
// LDS, store (or add, when K is split over workgroups) the 16 x 4U outputs, clear acc.
template <int U, int W, bool kCoherent = false>
__device__ __forceinline__ void stream_tile_end(float (&acc)[U][4], float *red, int wave, int tid, int lane,
                                                const TileRef &r, int64_t m0, int64_t M, int atomic)
{
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float v = acc[u][k];
            v = lane_group_sum(v);
            acc[u][k] = v;
        }
    if constexpr (W == 1) {
        if (lane < 16) {
            const int64_t n = r.lt * kTileRows + lane;
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int64_t m = m0 + 4 * u + k;
                    if (m < M && n < r.n) {
                        float *o = r.out + m * r.ldo + n;
                        if (atomic)
                            atomicAdd(o, acc[u][k]);
                        else
                            store_out<kCoherent>(o, acc[u][k]);
                    }
                }
        }
    } else {
        if (lane < 16) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    red[((wave * U + u) * 4 + k) * 16 + lane] = acc[u][k];
        }
        __syncthreads();
        for (int i = tid; i < U * 64; i += W * 64) {
            const int u = i >> 6, k = (i >> 4) & 3, c = i & 15;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w)
                v += red[((w * U + u) * 4 + k) * 16 + c];
            const int64_t m = m0 + 4 * u + k, n = r.lt * kTileRows + c;
            if (m < M && n < r.n) {
                float *o = r.out + m * r.ldo + n;
                if (atomic)
                    atomicAdd(o, v);
                else
                    store_out<kCoherent>(o, v);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k)
            acc[u][k] = 0.0f;
}

} // namespace
