// Chained projections for decode-sized M (1..4 tokens): up to MAMBO_MAX_CHAIN grouped
// launches of the block-diagonal weight-streaming kernel (gemm_stream_kernel, iq3s_gemm.hip)
// in ONE kernel launch, in order.
//
// Why: at one to four tokens a Llama decode step is hundreds of short launches (the 70B
// step: 320 launches of 2-200 MB of weights). Each pays the gap between kernels, the ramp
// of its first workgroups and the drain of its last ones, with HBM partly idle during
// each. Here the workgroups of launch L+1 are dispatched while launch L drains: each
// issues the loads of its first weight blocks at once (weights depend on no activation),
// and only then waits for launch L to finish before it stages its activations.
//
// Work: exactly the stream kernel's. Workgroup g of the grid belongs to the launch whose
// range of workgroups holds g (launches in order, `tpw` 16-row tiles per workgroup); its W
// waves split each tile's K blocks (wave w takes blocks w, w + W, ...) with the same
// per-tile arithmetic and cross-wave reduction order, so every output is bit-identical
// to the stream kernel's with the same W and no K split. Short workgroups, refilled by the
// hardware as others finish, keep uneven progress from stretching a launch: a persistent
// form (a fixed grid walking tiles round-robin) measured 2.2x slower on the 70B sweep,
// its slowest workgroups setting every launch's end (tile times p90 3x the median).
//
// Order (the semantics of `count` grouped launches on one stream): launch L's activation
// reads begin only after every output of launch L-1 is stored. Device counters in the
// caller's sync words carry this, with no address that every workgroup touches (one
// device-scope atomic on a single address costs ~25 ns, serialised: with one per
// workgroup the 70B sweep ran 4.5 times slower; spread over 32 lines, 1.6%):
//  * a workgroup waits for its output stores to complete (vmcnt 0), then adds one to the
//    line counter done1[g mod 32][L];
//  * the workgroup whose add completes a line (it knows from the returned count) adds one
//    to the launch counter done2[L]; the one whose add completes that (all lines of L) is
//    the launch's completer: it sets the 32 copies of flag[L], one per line, and clears
//    done1[*][L], done2[L] and flag[*][L-1] (every waiter of L-1 belongs to L, and all of
//    L's workgroups are done). The last launch sets no flag: nobody in the call waits on
//    it. So each call leaves the sync words zero for the next (graph replays included);
//  * a workgroup of launch L+1 polls its own copy flag[g mod 32][L] (one lane, agent-
//    scope loads, s_sleep between polls), then a workgroup barrier.
// Every earlier launch is then complete too (each of L's workgroups waited for L-1). So a
// launch may take as its activations the f32 outputs of an earlier launch of the chain,
// quantized to MXFP8 in its prologue (x_dtype f32/bf16), as a layer reads the output of
// the one before.
// Progress: the hardware dispatches the workgroups of a kernel in index order on each XCD,
// so a workgroup of launch L+1 is dispatched only after every workgroup of launch L on its
// XCD, and the workgroups it waits for are running or done, never queued behind it. Every
// wait is still bounded (s_memrealtime ticks): a workgroup that times out sets the status
// word and goes on (the outputs are then undefined), so the kernel always drains;
// mambo_chain_status reports it.
// Coherence across the 8 XCDs (each with its own L2) rides on the accesses, not on
// cache-wide maintenance: outputs are stored at device scope (global_store sc1, written
// through), rows quantized in the kernel are loaded at device scope (buffer_load sc1, never
// from a stale L1 or L2 copy), and a writer only waits for its own stores before its
// counter add. Agent-scope release/acquire fences (buffer_wbl2 / buffer_inv sc1, a
// writeback or invalidate of a whole L2) measured ~60 us per launch switch. MXFP8 inputs
// are never written inside a chain (it writes only f32), so their staging copies keep the
// plain policy.
#include "iq3s_stream.h"

namespace {

constexpr int kMaxChain = MAMBO_MAX_CHAIN;
// Sync words: 32 lines of 256 bytes of line counters (done1[x][L] at 64x + L), 32 lines of
// flag copies (flag[x][L] at kSyncFlag + 64x + L), the launch counters (done2[L] at
// kSyncDone2 + L) and the status word, each group in lines of its own.
constexpr int kSyncLines = 32;
constexpr int kSyncLineWords = 64;
constexpr int kSyncFlag = kSyncLines * kSyncLineWords;
constexpr int kSyncDone2 = 2 * kSyncLines * kSyncLineWords;
constexpr int kSyncStatus = kSyncDone2 + kSyncLineWords;
static_assert(kMaxChain <= kSyncLineWords && kSyncStatus < MAMBO_CHAIN_SYNC_WORDS, "sync words");
// Workgroups of a launch whose index g has g mod 32 == x.
__device__ __forceinline__ uint32_t chain_line_target(int wg0, int wgs, int x)
{
    const int first = wg0 + ((x - wg0) % kSyncLines + kSyncLines) % kSyncLines;
    return first >= wg0 + wgs ? 0u : (uint32_t)((wg0 + wgs - 1 - first) / kSyncLines + 1);
}
constexpr uint32_t kStatusTimeout = 1u;
// Ticks of the 100 MHz real-time counter (s_memrealtime) per microsecond.
constexpr uint64_t kTicksPerUs = 100;
// Cache policy of device-scope loads (CPol SC1).
constexpr int kDeviceScope = 16;

// One launch of the chain as the kernel reads it (kernel arguments; indexed by the
// wave-uniform launch number, so the fields are scalar loads from the argument segment).
struct ChainLaunchArgs {
    const uint8_t *x;  // MXFP8 values, or f32/bf16 rows
    const uint8_t *xs; // E8M0 scales (MXFP8)
    int64_t ldx;       // row stride of x in elements
    int64_t ldxs;
    const uint8_t *packed[kMaxGroup];
    float *out[kMaxGroup];
    int64_t ldo[kMaxGroup];
    int32_t n[kMaxGroup];
    int32_t tile_begin[kMaxGroup]; // first tile of projection g within the launch
    int32_t count, blocks, dtype;  // dtype: MAMBO_DTYPE_*
    int32_t tiles, wg0, wgs;       // its tiles; its first workgroup and workgroup count
};

struct ChainArgs {
    ChainLaunchArgs l[kMaxChain];
    uint32_t *sync;
    uint64_t timeout; // ticks per wait
    int32_t launches, m, kmax, tpw;
    uint32_t bias; // added to every wait target (tests force timeouts with it)
};
static_assert(sizeof(ChainArgs) <= 4096, "kernel arguments");

// Tile lt of a launch: its weights, output, N, row stride and tile within the projection
// (the launch's GroupArgs role in the stream kernel).
__device__ __forceinline__ TileRef chain_tile_ref(const ChainLaunchArgs &c, int64_t lt)
{
    TileRef r = {c.packed[0], c.out[0], (int64_t)c.n[0], c.ldo[0], lt};
#pragma unroll
    for (int g = 1; g < kMaxGroup; ++g)
        if (g < c.count && lt >= c.tile_begin[g]) {
            r.w = c.packed[g];
            r.out = c.out[g];
            r.n = c.n[g];
            r.ldo = c.ldo[g];
            r.lt = lt - c.tile_begin[g];
        }
    r.w += r.lt * (int64_t)c.blocks * kTileBytes;
    return r;
}

// Lane 0 of wave 0: wait until *p >= target, at most `timeout` ticks. Agent-scope atomic
// loads (vector memory), about 0.1 us of s_sleep between polls. Returns false on timeout.
#ifndef MAMBO_CHAIN_NAP
#define MAMBO_CHAIN_NAP 4
#endif
__device__ __forceinline__ bool chain_wait(const uint32_t *p, uint32_t target, uint64_t timeout)
{
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        __builtin_amdgcn_s_sleep(MAMBO_CHAIN_NAP);
        if (__builtin_amdgcn_s_memrealtime() - t0 > timeout)
            return false;
    }
    return true;
}

// One 32-element group of f32 or bf16 row data at byte `off` past the resource base, read
// at device scope: rows written earlier in the same kernel by another XCD's workgroups
// are read from where those stores went, never from a stale cache copy.
template <bool kBf16>
__device__ __forceinline__ void load_group32_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&v)[32])
{
    if constexpr (kBf16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const auto w = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16u * i, 0, kDeviceScope);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
                v[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const auto w = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16u * i, 0, kDeviceScope);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                v[4 * i + j] = __uint_as_float(w[j]);
        }
    }
}

// Move to the next (tile, step) pair of the workgroup's run unless at the last one (the
// ring's tail keeps re-reading it); `c` as the stream kernel's cursor.
__device__ __forceinline__ void chain_advance(StreamCursor &c, int total, int steps, const ChainLaunchArgs &l)
{
    if (c.s + 1 < total) {
        ++c.s;
        if (++c.i == steps) {
            c.i = 0;
            ++c.t;
            c.w = byte_rsrc(chain_tile_ref(l, c.t).w);
        }
    }
}

// kQuant: the chain has launches with f32/bf16 rows to quantize (the build without it
// keeps the 32 values of a group out of the register budget).
template <int W, int kLg, bool kQuant>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2))) void gemm_chain_kernel(ChainArgs a)
{
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ __align__(16) uint32_t s_grid[512 << kLg];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, q = lane >> 4;
    const int rows = a.m;
    const StreamLds Ld = stream_lds(1, W, rows, a.kmax, true);
    const uint8_t *lut = reinterpret_cast<const uint8_t *>(s_grid);
    const uint32_t c4 = 4u * (uint32_t)(lane & ((1 << kLg) - 1));

    // this workgroup's launch and run of tiles
    const int g = blockIdx.x;
    int L = 0;
    while (L + 1 < a.launches && g >= a.l[L + 1].wg0)
        ++L;
    const ChainLaunchArgs &c = a.l[L];
    const int B = c.blocks, K = B * 256;
    const int t_begin = (g - c.wg0) * a.tpw;
    const int ntw = min(a.tpw, c.tiles - t_begin);
    const int steps = (B + W - 1) / W;
    const int total = ntw * steps;

    // The first look at launch L-1's flag goes out before anything else: vector memory
    // completes in issue order, so reading it then waits for that load alone, not for the
    // weights issued after it, and a workgroup whose dependency is already met stages its
    // rows one round trip after its start, while its first weights are still in flight.
    const uint32_t *flag = a.sync + kSyncFlag + kSyncLineWords * (g % kSyncLines) + (L - 1);
    uint32_t seen = 0u;
    if (L > 0 && tid == 0)
        seen = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_sched_barrier(0);
    // codebook (direct copies into LDS), then the ring's first weight loads: both go out
    // before any wait, so a workgroup of launch L+1 streams its weights while L drains
    {
        const __amdgpu_buffer_rsrc_t gr = byte_rsrc(rep_grid<kLg>());
        if constexpr (kLg == 0) {
            for (int i = wave; i < 8; i += W)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (lds_ptr)(s_grid + 64 * i), 4, 4u * lane, 256u * i, 0, 0);
        } else {
            for (int i = wave; i < stream_lut_bytes(kLg) / 1024; i += W)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(gr, (lds_ptr)(s_grid + 256 * i), 16, 16u * lane, 1024u * i, 0,
                                                         0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    WTile wr[kDepth];
    StreamCursor pc = {0, 0, t_begin, byte_rsrc(chain_tile_ref(c, t_begin).w)};
#pragma unroll
    for (int j = 0; j < kDepth - 1; ++j) {
        wr[j] = load_w_rsrc(pc.w, (uint32_t)min(wave + pc.i * W, B - 1) * kTileBytes, lane, col);
        chain_advance(pc, total, steps, c);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (tid < 20)
        reinterpret_cast<uint32_t *>(smem + Ld.zero)[tid] = tid < 16 ? 0u : 0x7F7F7F7Fu;

    // launch L-1 done: every one of its workgroups stored its outputs
    if (L > 0) {
        if (tid == 0) {
            const bool ok = seen >= 1u + a.bias || chain_wait(flag, 1u + a.bias, a.timeout);
            if (!ok)
                __hip_atomic_fetch_or(a.sync + kSyncStatus, kStatusTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
    // this launch's activation rows into LDS
    if (!kQuant || c.dtype == MAMBO_DTYPE_MXFP8) {
        // rows as 16-byte chunks (K is a multiple of 256, so none straddles rows; slot e of
        // row r takes chunk act_slot(e, r)), their scales as dwords (the host requires
        // 4-byte aligned scale rows)
        const int nx = rows * K / 16;
        const __amdgpu_buffer_rsrc_t xr = byte_rsrc(c.x);
        for (int i = wave; 64 * i < nx; i += W) {
            const int e = 64 * i + lane, r = e * 16 / K;
            if (e < nx)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(smem + Ld.x + 1024 * i), 16,
                                                         (uint32_t)(r * c.ldx + 16 * act_slot(e - r * (K / 16), r)),
                                                         0, 0, 0);
        }
        const int ns = rows * (K / 128);
        const __amdgpu_buffer_rsrc_t sr = byte_rsrc(c.xs);
        for (int i = wave; 64 * i < ns; i += W) {
            const int e = 64 * i + lane, r = e / (K / 128);
            if (e < ns)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(smem + Ld.xs + 256 * i), 4,
                                                         (uint32_t)(r * c.ldxs + 4 * (e - r * (K / 128))), 0, 0, 0);
        }
    } else {
        // f32 / bf16 rows (16-byte aligned): MXFP8 with the quantizer's arithmetic, one
        // 32-element group per thread
        const int gpr = K / 32, groups = rows * gpr;
        const __amdgpu_buffer_rsrc_t xr = byte_rsrc(c.x);
        for (int gi = tid; gi < groups; gi += W * 64) {
            const int r = gi / gpr, gg = gi - r * gpr;
            float v[32];
            if (c.dtype == MAMBO_DTYPE_BF16)
                load_group32_coherent<true>(xr, (uint32_t)(2 * (r * c.ldx + 32 * gg)), v);
            else
                load_group32_coherent<false>(xr, (uint32_t)(4 * (r * c.ldx + 32 * gg)), v);
            uint32_t codes[8];
            const int scale = quantize_group32(v, codes);
            uint4 *dst = reinterpret_cast<uint4 *>(smem + Ld.x + r * K + 16 * act_slot(2 * gg, r));
            dst[0] = uint4{codes[0], codes[1], codes[2], codes[3]};
            dst[1] = uint4{codes[4], codes[5], codes[6], codes[7]};
            smem[Ld.xs + r * gpr + gg] = (uint8_t)scale;
        }
    }
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); // vmcnt(0): codebook and row copies
    __syncthreads();

    // block-diagonal operand of the rows (see gemm_stream_kernel)
    ALane al[1];
    {
        const int r = lane & 3;
        al[0] = a_lane<true>(lane, r < rows, smem + Ld.x + r * K, smem + Ld.xs + r * (K / 32), smem + Ld.zero,
                       smem + Ld.zero + 64);
    }
    float acc[1][4] = {{0.0f, 0.0f, 0.0f, 0.0f}};
    float *red = reinterpret_cast<float *>(smem + Ld.red);
    int ci = 0, tile_no = 0;
    for (int s0 = 0; s0 < total; s0 += kDepth) {
#pragma unroll
        for (int jj = 0; jj < kDepth; ++jj) {
            const int s = s0 + jj;
            const int slot = (jj + kDepth - 1) % kDepth;
            wr[slot] = load_w_rsrc(pc.w, (uint32_t)min(wave + pc.i * W, B - 1) * kTileBytes, lane, col);
            chain_advance(pc, total, steps, c);
            if constexpr (MAMBO_SCHED_FENCE)
                __builtin_amdgcn_sched_barrier(0);
            if (s < total) {
                const int blk = wave + ci * W;
                ATile<1> at;
                load_a<1>(at, al, min(blk, B - 1), smem + Ld.zero);
                __builtin_amdgcn_sched_barrier(0); // activation reads before the codebook reads
                compute_block<1, kLg>(wr[jj], at, lut, c4, acc, blk < B);
                if (++ci == steps) {
                    stream_tile_end<1, W, true>(acc, red + (tile_no & 1) * (W * 64), wave, tid, lane,
                                                chain_tile_ref(c, t_begin + tile_no), 0, rows, 0);
                    ci = 0;
                    ++tile_no;
                }
            }
            if constexpr (MAMBO_SCHED_FENCE)
                __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Wave 0 stored every output of the run (the tile-end sums, at device scope): once
    // they are complete (vmcnt 0), count the workgroup in (see the protocol above).
    if (wave == 0) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        uint32_t completer = 0u;
        if (lane == 0) {
            const int x = g % kSyncLines;
            const uint32_t line = __hip_atomic_fetch_add(a.sync + kSyncLineWords * x + L, 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            if (line + 1u == chain_line_target(c.wg0, c.wgs, x)) {
                const uint32_t lines = __hip_atomic_fetch_add(a.sync + kSyncDone2 + L, 1u, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
                completer = lines + 1u == (uint32_t)min(c.wgs, kSyncLines) ? 1u : 0u;
            }
        }
        if (__builtin_amdgcn_readfirstlane(completer)) {
            // every workgroup of L has counted in: clear L's counters and L-1's flags, then
            // raise L's flags (but for the last launch, which no one in the call waits on)
            if (lane < kSyncLines) {
                __hip_atomic_store(a.sync + kSyncLineWords * lane + L, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (L > 0)
                    __hip_atomic_store(a.sync + kSyncFlag + kSyncLineWords * lane + (L - 1), 0u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            } else if (lane == kSyncLines) {
                __hip_atomic_store(a.sync + kSyncDone2 + L, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (L + 1 < a.launches && lane < kSyncLines)
                __hip_atomic_store(a.sync + kSyncFlag + kSyncLineWords * lane + L, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int W, int kLg, bool kQuant>
void chain_launch(unsigned grid, size_t lds, hipStream_t s, const ChainArgs &a)
{
    MAMBO_LAUNCH((gemm_chain_kernel<W, kLg, kQuant>), dim3(grid), dim3(W * 64), lds, s, a);
}

// The builds: waves 4, 8, 16 x codebook copies 1, 4, 16 (x in-kernel quantization).
void chain_dispatch(int w, int lg, bool quant, unsigned grid, size_t lds, hipStream_t s, const ChainArgs &a)
{
#define MAMBO_C(WV, LG)                                                                                            \
    if (w == WV && lg == LG)                                                                                       \
        return quant ? chain_launch<WV, LG, true>(grid, lds, s, a) : chain_launch<WV, LG, false>(grid, lds, s, a);
    MAMBO_C(4, 0) MAMBO_C(4, 2) MAMBO_C(4, 4) MAMBO_C(8, 0) MAMBO_C(8, 2) MAMBO_C(8, 4) MAMBO_C(16, 0)
    MAMBO_C(16, 2) MAMBO_C(16, 4)
#undef MAMBO_C
}

// LDS per CU on gfx950.
constexpr int kChainLdsPerCU = 160 * 1024;

// Codebook copies (log2) for `m` tokens (as the stream kernel on K >= 8192).
int chain_copies_lg(int64_t m) { return m == 1 ? 0 : m == 2 ? 2 : 4; }

} // namespace

extern "C" int mambo_iq3s_fp8_matmul_chain(int64_t m, const mambo_chain_launch *launches, int count,
                                           const mambo_chain_config *cfg, uint32_t *sync, mambo_stream_t stream)
{
    MAMBO_REQUIRE(launches && sync, MAMBO_ERR_VALUE, "null pointer");
    MAMBO_REQUIRE(count >= 1 && count <= kMaxChain, MAMBO_ERR_VALUE, "count must be in [1, %d] (got %d)", kMaxChain,
                  count);
    MAMBO_REQUIRE(m >= 1 && m <= 4, MAMBO_ERR_VALUE, "chained projections take 1..4 tokens (got M=%lld)",
                  (long long)m);
    MAMBO_REQUIRE((uintptr_t)sync % 4 == 0, MAMBO_ERR_VALUE, "sync words must be 4-byte aligned");
    const int waves = cfg && cfg->waves ? cfg->waves : 4;
    MAMBO_REQUIRE(waves == 4 || waves == 8 || waves == 16, MAMBO_ERR_VALUE, "chain waves must be 4, 8 or 16 (got %d)",
                  waves);
    const int tpw = cfg && cfg->tiles_per_workgroup ? cfg->tiles_per_workgroup : 1;
    MAMBO_REQUIRE(tpw >= 1 && tpw <= 4096, MAMBO_ERR_VALUE, "tiles per workgroup must be in [1, 4096] (got %d)", tpw);
    ChainArgs a = {};
    int64_t wgs = 0, kmax = 0;
    bool quant = false;
    for (int L = 0; L < count; ++L) {
        const mambo_chain_launch &cl = launches[L];
        ChainLaunchArgs &d = a.l[L];
        MAMBO_REQUIRE(cl.x, MAMBO_ERR_VALUE, "launch %d: null activations", L);
        MAMBO_REQUIRE(cl.count >= 1 && cl.count <= kMaxGroup, MAMBO_ERR_VALUE,
                      "launch %d: count must be in [1, %d] (got %d)", L, kMaxGroup, cl.count);
        MAMBO_REQUIRE(cl.blocks >= 1 && cl.blocks <= (1 << 20), MAMBO_ERR_VALUE, "launch %d: bad K blocks %lld", L,
                      (long long)cl.blocks);
        const int64_t k = cl.blocks * 256;
        MAMBO_REQUIRE(cl.ldx >= k && cl.ldx < ((int64_t)1 << 27), MAMBO_ERR_VALUE,
                      "launch %d: activation row stride must cover the row (and be below 2^27)", L);
        if (cl.x_dtype == MAMBO_DTYPE_MXFP8) {
            MAMBO_REQUIRE(cl.xs, MAMBO_ERR_VALUE, "launch %d: null activation scales", L);
            MAMBO_REQUIRE((uintptr_t)cl.x % 16 == 0 && cl.ldx % 16 == 0, MAMBO_ERR_VALUE,
                          "launch %d: x_values base and row stride must be 16-byte aligned", L);
            MAMBO_REQUIRE(cl.ldxs >= k / 32 && cl.ldxs < ((int64_t)1 << 27), MAMBO_ERR_VALUE,
                          "launch %d: scale row stride must cover the row", L);
            MAMBO_REQUIRE((uintptr_t)cl.xs % 4 == 0 && cl.ldxs % 4 == 0, MAMBO_ERR_VALUE,
                          "launch %d: x_scales base and row stride must be 4-byte aligned", L);
        } else {
            MAMBO_REQUIRE(cl.x_dtype == MAMBO_DTYPE_F32 || cl.x_dtype == MAMBO_DTYPE_BF16, MAMBO_ERR_VALUE,
                          "launch %d: x_dtype must be MXFP8, float32 or bfloat16", L);
            const int64_t esz = cl.x_dtype == MAMBO_DTYPE_BF16 ? 2 : 4;
            MAMBO_REQUIRE((uintptr_t)cl.x % 16 == 0 && (cl.ldx * esz) % 16 == 0, MAMBO_ERR_VALUE,
                          "launch %d: activation rows must be 16-byte aligned", L);
            quant = true;
        }
        d.x = reinterpret_cast<const uint8_t *>(cl.x);
        d.xs = cl.xs;
        d.ldx = cl.ldx;
        d.ldxs = cl.ldxs;
        d.count = cl.count;
        d.blocks = (int32_t)cl.blocks;
        d.dtype = cl.x_dtype;
        int64_t lt = 0;
        for (int g = 0; g < cl.count; ++g) {
            const mambo_projection &p = cl.proj[g];
            MAMBO_REQUIRE(p.packed && p.out, MAMBO_ERR_VALUE, "launch %d projection %d: null pointer", L, g);
            MAMBO_REQUIRE(p.n >= 1 && p.n <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "launch %d projection %d: bad N", L, g);
            MAMBO_REQUIRE(p.ldo >= p.n, MAMBO_ERR_VALUE, "launch %d projection %d: output row stride must cover the row",
                          L, g);
            MAMBO_REQUIRE((uintptr_t)p.packed % 16 == 0, MAMBO_ERR_VALUE,
                          "launch %d projection %d: packed weight must be 16-byte aligned", L, g);
            d.packed[g] = p.packed;
            d.out[g] = p.out;
            d.n[g] = (int32_t)p.n;
            d.ldo[g] = p.ldo;
            d.tile_begin[g] = (int32_t)lt;
            lt += (p.n + kTileRows - 1) / kTileRows;
        }
        const int64_t lw = (lt + tpw - 1) / tpw;
        MAMBO_REQUIRE(lt <= 0x7FFFFFFF && wgs + lw <= 0x7FFFFFFF, MAMBO_ERR_VALUE, "chain too large for one launch");
        d.tiles = (int32_t)lt;
        d.wg0 = (int32_t)wgs;
        d.wgs = (int32_t)lw;
        wgs += lw;
        kmax = std::max(kmax, k);
    }
    const int lg = chain_copies_lg(m);
    const StreamLds Lds = stream_lds(1, waves, (int)m, (int)kmax, true);
    MAMBO_REQUIRE(Lds.total + stream_lut_bytes(lg) + 64 <= kChainLdsPerCU, MAMBO_ERR_VALUE,
                  "chain: %d tokens of K=%lld need %d bytes of LDS per workgroup", (int)m, (long long)kmax,
                  Lds.total + stream_lut_bytes(lg));
    const int64_t timeout_us = cfg && cfg->timeout_us ? cfg->timeout_us : 2000000;
    MAMBO_REQUIRE(timeout_us > 0 && timeout_us <= 60000000, MAMBO_ERR_VALUE, "chain: timeout must be in (0, 60 s]");
    a.sync = sync;
    a.timeout = (uint64_t)timeout_us * kTicksPerUs;
    a.launches = count;
    a.m = (int32_t)m;
    a.kmax = (int32_t)kmax;
    a.tpw = tpw;
    a.bias = cfg ? (uint32_t)cfg->wait_bias : 0u;
    chain_dispatch(waves, lg, quant, (unsigned)wgs, (size_t)Lds.total, (hipStream_t)stream, a);
    return mambo_check_launch("iq3s_fp8_matmul_chain");
}

extern "C" int mambo_chain_status(uint32_t *sync)
{
    MAMBO_REQUIRE(sync, MAMBO_ERR_VALUE, "null pointer");
    static thread_local uint32_t words[MAMBO_CHAIN_SYNC_WORDS];
    hipError_t err = hipMemcpy(words, sync, sizeof(words), hipMemcpyDeviceToHost);
    if (err != hipSuccess)
        return mambo_fail(MAMBO_ERR_RUNTIME, "chain status: %s", hipGetErrorString(err));
    const uint32_t status = words[kSyncStatus];
    bool counters_clear = true;
    for (int i = 0; i < kSyncStatus; ++i)
        counters_clear = counters_clear && words[i] == 0u;
    if (status != 0u) {
        // after a timeout, launches may have completed out of order and left flags raised:
        // clear every word, so the next call starts from zero
        for (uint32_t &w : words)
            w = 0u;
        err = hipMemcpy(sync, words, sizeof(words), hipMemcpyHostToDevice);
        if (err != hipSuccess)
            return mambo_fail(MAMBO_ERR_RUNTIME, "chain status: %s", hipGetErrorString(err));
        return mambo_fail(MAMBO_ERR_RUNTIME, "chained projections: a dependency wait timed out; outputs are "
                                             "undefined (the sync words are cleared)");
    }
    if (!counters_clear)
        return mambo_fail(MAMBO_ERR_RUNTIME, "chain sync words are not clear (a chain is still running on them, or "
                                             "they were not zero before the first call)");
    return MAMBO_OK;
}
