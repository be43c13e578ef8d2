// mfma_staged: the prefill GEMM for gfx950, C[M,N] = A[M,K] * W[N,K]^T with
// BF16/FP16 inputs, fp32 accumulation and a bf16/fp16/fp32 epilogue.
//
// This is the "staged" rung of the reference ladder
// (cuda_kernels/gemm/src/gemm_bench.cu:117-196, gemm_wmma.cu:116-207)
// designed for CDNA4 instead of translated:
//   * 128 x 128 macro tile per 256-thread workgroup (4 waves in a 2x2
//     grid, 64 x 64 each), K-tiles of 64 elements; grids with enough
//     128 x 256 tiles for every CU take those (8 waves in a 2x4 grid, 64 x
//     64 each), grids of at most 128 tiles of 128 x 128 (half the CUs) take
//     64 x 64 tiles (waves of 32 x 32), and fp32 logits over a W larger
//     than the Infinity Cache take 256 x 256 tiles (8 waves of 128 x 64, the
//     fp32 C tile leaving LDS in two passes of 128 rows);
//   * operands move global -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging) into a ring of STAGES tile buffers; tiles t+1 .. t+STAGES-1
//     are in flight while tile t is multiplied, and each wave waits on its
//     own vmcnt for exactly the tile it needs before the one barrier per
//     K-tile;
//   * with a 3-deep ring and one workgroup per CU (SP = 1) the copies of
//     tile t+2 are spread between the MFMAs of tile t instead of issued as
//     one burst after the barrier: a copy instruction that finds the CU's
//     load queue full holds up every later instruction of its wave, MFMAs
//     included, so a burst leaves the matrix units idle while the queue
//     drains;
//   * LDS rows of 64 elements are 8 chunks of 16 bytes; chunk c of row r
//     sits at position c ^ ((r >> 1) & 7).  gfx950's LDS serves 16 lanes of
//     a ds_read_b128 per clock from 64 banks (256 bytes), and with this key
//     the 16 rows one MFMA fragment read touches per clock land in 16
//     distinct 16-byte bank groups (rows r and r+8 no longer collide);
//   * v_mfma_f32_32x32x16_{bf16,f16} with W as the first operand and A as
//     the second, so each lane ends with 4 consecutive output columns per
//     accumulator quad and stores them with one 8- or 16-byte write;
//   * XCD-aware tile order so the tiles that share A and W rows run on the
//     same XCD's L2.
// Rows past M or N are clamped for loading and masked at the store; K-tail
// chunks (K must be a multiple of 8) are copied from a zero chunk in device
// memory, so the LDS tile is zero past K.
#include <type_traits>

#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kBK = 64;        // K elements per tile = 8 chunks of 16 bytes
constexpr int kChunks = kBK / 8;
constexpr int kLdsPerCu = 160 * 1024;   // LDS bytes of one CU (gfx950)

// Source of the K-tail chunks: 16 zero bytes in global memory.
__device__ u32x4_t g_zero_chunk = {0u, 0u, 0u, 0u};

__device__ __forceinline__ int lds_swizzle(int row) { return (row >> 1) & 7; }

// B[K,N] stages: k-row r of the W part holds its 16-byte column chunks in
// position chunk ^ kn_swizzle(r).  A transposing fragment read touches 8
// k-rows (r, r+1, r+2, r+3, r+8, ..., r+11) x 64 bytes; flipping bits 2-3
// of the chunk position by r % 4 (by bit 1 of r with 8 chunks per row,
// whose rows alternate between two 128-byte halves of the banks) puts two
// of those rows in each quarter of the 64 banks.
template <int BN>
__device__ __forceinline__ int kn_swizzle(int r) {
    if constexpr (BN >= 128) return (r & 3) << 2;
    else return ((r >> 1) & 1) << 2;
}


// RS: output row i is multiplied by row_scale[i] before rounding (with
// EPI_NONE or EPI_SILU_MUL, where it scales both sums of a pair).
// SP: copy schedule.  0: each K-tile's copies as one burst after the
// barrier; 1: spread between the MFMAs (3-deep ring only).
// KN: B is given as B[K,N] (row stride ldb >= N, N a multiple of 8); the W
// part of a stage then holds 64 k-rows of BN columns, copied as they lie in
// memory, and the W fragments are read with gfx950's transposing LDS read.
template <int DT, int DT_OUT, int BM, int BN, int WGM, int WGN, int STAGES, int EPI, int RS, int SP, int KN = 0>
__global__ __launch_bounds__(WGM * WGN * 64) void mfma_staged_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, int64_t m, int64_t n, int64_t k, int64_t lda,
    int64_t ldb, void* __restrict__ c, int64_t ldc, int c_vec, uint64_t* __restrict__ keys,
    const float* __restrict__ row_scale, SampleArgs sa) {
    // The arguments the copies need first (a, w, m, n, k, lda, ldb: 56
    // bytes) lead the list, so with kernel-argument preloading (14 SGPRs)
    // the first K-tiles are requested before any argument load returns;
    // the grid shape is recomputed here rather than passed.
    constexpr int NW = WGM * WGN;        // waves, in a WGM x WGN grid
    constexpr int NT = NW * 64;          // threads
    constexpr int WM = BM / WGM;         // wave tile rows (M)
    constexpr int WN = BN / WGN;         // wave tile cols (N)
    constexpr int MJ = WM / 32;          // 32-row blocks of A per wave
    constexpr int NI = WN / 32;          // 32-row blocks of W per wave
    constexpr int ROWS = BM + BN;        // LDS rows per stage (A rows, then W rows)
    constexpr int IPW = ROWS / (8 * NW); // DMA instructions per wave per tile (8 rows each)
    constexpr int AHEAD = STAGES - 1;    // tiles in flight ahead of the one multiplied
    static_assert(IPW * 8 * NW == ROWS && WM % 32 == 0 && WN % 32 == 0, "tile shape");
    static_assert(AHEAD >= 1 && AHEAD <= 3 && AHEAD * IPW < 64, "vmcnt range");
    static_assert(SP != 1 || STAGES == 3, "the spread schedule refills the stage of tile t - 1 with tile t + 2");
    // EPI_SILU_MUL: the W rows of a tile alternate 32 gate rows and the 32 up
    // rows of the same output columns, so block pair (2i, 2i + 1) of a wave
    // holds gate and up values of one 32-column group in the same lanes.
    static_assert(EPI != EPI_SILU_MUL || NI % 2 == 0, "gate/up pairs per wave");
    static_assert(!RS || EPI != EPI_ARGMAX, "row scale with a stored output");
    static_assert(!KN || (EPI == EPI_NONE && !RS && (SP == 0 || SP == 1)), "B[K,N]: plain GEMM, copy schedules");
    constexpr int BNO = EPI == EPI_SILU_MUL ? BN / 2 : BN;   // output columns per tile

    // LDS: the ring of K-tile stages, reused after the K loop for the C tile.
    // A C tile larger than a CU's LDS (256 x 256 with fp32 output) goes out
    // in EPASS passes of EP_ROWS rows, one row of the wave grid per pass.
    constexpr int OB = DT_OUT == NANOVLLM_GEMM_F32 ? 4 : 2;     // output bytes
    constexpr int PITCH = BNO * OB + 16;                         // C-tile row pitch in LDS
    constexpr int STAGE_CHUNKS = ROWS * kChunks;
    constexpr int RING_BYTES = STAGES * STAGE_CHUNKS * 16;
    constexpr int EP_ROWS = BM * PITCH <= kLdsPerCu ? BM : WM;
    constexpr int EPASS = BM / EP_ROWS;
    static_assert(EP_ROWS * PITCH <= kLdsPerCu && RING_BYTES <= kLdsPerCu, "LDS per CU");
    static_assert(EPASS == 1 || EPI == EPI_NONE, "C-tile passes: plain store only");
    constexpr int LDS_BYTES = RING_BYTES > EP_ROWS * PITCH ? RING_BYTES : EP_ROWS * PITCH;
    __shared__ u32x4_t ring[LDS_BYTES / 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN;
    const int wn = wave % WGN;
    const int half = lane >> 5;
    const int r32 = lane & 31;

    // The epilogue's arguments are loaded before the K loop (right after the
    // first copies are issued, so their load overlaps those copies): a
    // scalar load still in flight inside the K loop shares the LDS counter
    // with the fragment reads and completes out of order, which would turn
    // every fragment wait into lgkmcnt(0).
    auto hold_epilogue_args = [&] {
        asm volatile("" :: "s"(c), "s"(ldc), "s"(c_vec), "s"(m), "s"(n), "s"(keys), "s"(row_scale));
    };

    const int tiles_m = static_cast<int>((m + BM - 1) / BM);
    const int tiles_n = static_cast<int>((n + BNO - 1) / BNO);
    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int64_t m0 = int64_t(tm) * BM;
    const int64_t n0 = int64_t(tn) * BNO;   // first output column

    // DMA instruction j of this wave fills LDS rows 8 i .. 8 i + 7 of a stage,
    // i = wave * IPW + j; lane L writes row 8 i + L / 8, position L % 8, which
    // holds logical chunk (L % 8) ^ swizzle(row).
    //
    // KN: instruction i >= BM / 8 copies chunks q = 64 (i - BM / 8) + L of the
    // W part instead, k-row q / (BN / 8), position q % (BN / 8), which holds
    // logical chunk (8 columns) position ^ swizzle_kn(row).  kpos[j] is the
    // k position the instruction's chunk starts at (chunk offset in an A row,
    // k-row of B; K for a B chunk past N, which is then always the zero
    // chunk), kn_row[j] whether it advances by rows of B.
    const uint16_t* src[IPW];
    int koff[IPW];
    int kpos[IPW];
    bool kn_row[IPW];
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int row = 8 * (wave * IPW + j) + (lane >> 3);
        const int chunk = (lane & 7) ^ lds_swizzle(row);
        koff[j] = chunk * 8;
        kpos[j] = koff[j];
        kn_row[j] = false;
        if (KN && row >= BM) {
            constexpr int CPRB = BN / 8;   // chunks per k-row of the W part
            const int q = 64 * (wave * IPW + j - BM / 8) + lane;
            const int kr = q / CPRB;
            const int64_t col = n0 + 8 * ((q % CPRB) ^ kn_swizzle<BN>(kr));
            const bool in = col < n;       // N % 8 == 0: a chunk is in or out whole
            src[j] = w + (in ? int64_t(kr) * ldb + col : 0);
            kpos[j] = in ? kr : int(k < INT32_MAX ? k : INT32_MAX);
            kn_row[j] = true;
        } else if (row < BM) {
            src[j] = a + min_i64(m0 + row, m - 1) * lda + koff[j];
        } else if constexpr (EPI == EPI_SILU_MUL) {
            const int wr = row - BM;
            const int64_t col = n0 + 32 * (wr >> 6) + (wr & 31);     // output column of this row
            src[j] = w + (((wr >> 5) & 1) ? n : 0) * ldb + min_i64(col, n - 1) * ldb + koff[j];
        } else {
            src[j] = w + min_i64(n0 + (row - BM), n - 1) * ldb + koff[j];
        }
    }

    // K-tiles are counted in 32 bits (the launcher checks k < 2^31), and the
    // ring stage of a tile advances without a division.
    const int ktiles = static_cast<int>((k + kBK - 1) / kBK);
    const uint32_t ring_lds = lds_address(ring);
    // Address of the zero chunk, held in registers for the whole kernel (in
    // position-independent code it is otherwise reloaded from the GOT by a
    // scalar load at every use).
    const void* zero = &g_zero_chunk;
    asm volatile("" : "+s"(zero));
    // Source of instruction j's chunk of the K-tile starting at k0.
    auto chunk_src = [&](int j, int64_t k0) -> const void* {
        if (k0 + kpos[j] >= k) return zero;
        return src[j] + (KN && kn_row[j] ? k0 * ldb : k0);
    };
    auto issue = [&](int t, int stage) {
        const int64_t k0 = int64_t(t) * kBK;
        const uint32_t dst = ring_lds + uint32_t(stage * STAGE_CHUNKS + 64 * wave * IPW) * 16u;
        if constexpr (KN) {
#pragma unroll
            for (int j = 0; j < IPW; ++j) dma16(chunk_src(j, k0), dst + 1024u * j);
        } else if (k0 + kBK <= k) {
#pragma unroll
            for (int j = 0; j < IPW; ++j) dma16(src[j] + k0, dst + 1024u * j);
        } else {
            // The last K-tile of a K that is not a multiple of 64.
#pragma unroll
            for (int j = 0; j < IPW; ++j)
                dma16(k0 + koff[j] < k ? static_cast<const void*>(src[j] + k0) : zero, dst + 1024u * j);
        }
    };

    // Copy instruction j of tile t into `stage` alone (the spread schedule).
    auto issue_one = [&](int t, int stage, int j) {
        const int64_t k0 = int64_t(t) * kBK;
        const uint32_t dst = ring_lds + uint32_t(stage * STAGE_CHUNKS + 64 * wave * IPW) * 16u + 1024u * j;
        dma16(chunk_src(j, k0), dst);
    };

    f32x16_t acc[NI][MJ];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j] = f32x16_t{};

    // Fragment rows: lane l reads row (base + l % 32) with base a multiple of
    // 32, so the swizzle key is ((l % 32) >> 1) & 7 = (l >> 1) & 7.
    const int swz = (lane >> 1) & 7;
    const int a_row0 = wm * WM + r32;
    const int w_row0 = BM + wn * WN + r32;

    // Two fragment register sets: the MFMAs of K-step kk run from one while
    // the ds_reads of kk + 1 fill the other.
    u32x4_t af0[MJ], wf0[NI], af1[MJ], wf1[NI];
    // KN: W fragment i of K-step kk is two ds_read_b64_tr_b16.  Within each
    // 16-lane group the instruction returns, to lane i, element i % 4 of the
    // 8 bytes lanes i / 4, i / 4 + 4, i / 4 + 8, i / 4 + 12 point at; lane j
    // of the group points at k-row (4 r + j / 4) and columns 4 (j % 4) .. +3
    // of its 16-column half, so lane l ends with k = 16 kk + 8 (l / 32) +
    // 4 r + 0..3 of column l % 32: the operand layout above, 4 k at a time.
    // The swizzle spreads the 8 k-rows one read touches over all 64 banks.
    constexpr int KN_PITCH = BN * 2;   // bytes per k-row of the W part
    const int kn_q = (lane & 15) >> 2;
    const uint32_t kn_row_off = uint32_t(8 * (lane >> 5) + kn_q) * KN_PITCH;
    uint32_t kn_col_off[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int col = wn * WN + 32 * i + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
        kn_col_off[i] = uint32_t(((col >> 3) ^ kn_swizzle<BN>(kn_q)) * 16 + (col & 7) * 2);
    }
    auto read_frags = [&](const u32x4_t* tile, int kk, u32x4_t (&af)[MJ], u32x4_t (&wf)[NI]) {
        const int chunk = (2 * kk + half) ^ swz;
#pragma unroll
        for (int j = 0; j < MJ; ++j) af[j] = tile[(a_row0 + 32 * j) * kChunks + chunk];
        if constexpr (KN) {
            typedef short v4i16_t __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) v4i16_t* lds_v4;
            const uint32_t wpart = lds_address(tile + BM * kChunks) + kn_row_off + uint32_t(16 * kk) * KN_PITCH;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t a0 = wpart + kn_col_off[i];
                const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4)(uintptr_t)a0);
                const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4)(uintptr_t)(a0 + 4 * KN_PITCH));
                const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
                wf[i] = u32x4_t{l2[0], l2[1], h2[0], h2[1]};
            }
        } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) wf[i] = tile[(w_row0 + 32 * i) * kChunks + chunk];
        }
    };
    auto mfmas = [&](const u32x4_t (&af)[MJ], const u32x4_t (&wf)[NI]) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < MJ; ++j) acc[i][j] = mfma_32x32x16<DT>(wf[i], af[j], acc[i][j]);
    };
    // Wait until tile u has landed in every wave's part of its stage (each
    // wave waits on its own vmcnt, the barrier covers the others), then
    // refill `free_stage`, the stage the previous tile used, with tile
    // u + AHEAD.
    auto tile_ready = [&](int u, int free_stage) {
        const int later = ktiles - 1 - u;   // tiles already issued after u, capped at AHEAD - 1
        if constexpr (AHEAD >= 3) {
            if (later >= 2) wait_vmcnt<2 * IPW>();
            else if (later == 1) wait_vmcnt<IPW>();
            else wait_vmcnt<0>();
        } else if constexpr (AHEAD == 2) {
            if (later >= 1) wait_vmcnt<IPW>();
            else wait_vmcnt<0>();
        } else {
            wait_vmcnt<0>();
        }
        // Every ds_read of the previous tile has returned before the barrier,
        // so the stage refilled below is free in every wave.  The copy burst
        // is issued at raised wave priority: with two workgroups per CU it
        // then enters the load queue ahead of the other workgroup's
        // instructions (2048 x 5120 x 1024: 30.3 / 30.2 -> 29.6 / 29.1 us,
        // 2304 x 5120 x 1024: 31.5 / 31.2 -> 30.9 / 30.5 us; raising it over
        // the MFMAs instead cost 4-10%).
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_setprio(3);
        if (u + AHEAD < ktiles) issue(u + AHEAD, free_stage);
        __builtin_amdgcn_s_setprio(0);
    };

    if constexpr (SP == 1) {
        // Tile t's K-steps 0, 1 and 2 each carry D0, D1, D2 of the wave's IPW
        // copy instructions for tile t + 2, which go to the stage tile t - 1
        // used (free since the barrier that opened tile t).  All IPW are out
        // before the wait for tile t + 1, so that wait is vmcnt <= IPW, and
        // tile t + 2 has the rest of tile t and all of tile t + 1 to land.
        constexpr int D0 = (IPW + 2) / 3, D1 = (IPW - D0 + 1) / 2, D2 = IPW - D0 - D1;
        constexpr int STEP = NI * MJ;   // MFMAs per K-step
        // The MFMAs of one K-step with copies J0 .. J0 + CNT - 1 of tile tt
        // evenly between them; the scheduling barriers pin each copy to its
        // slot in the MFMA sequence.
        auto mfmas_copy = [&](const u32x4_t (&af)[MJ], const u32x4_t (&wf)[NI], int tt, int stage, auto j0_c,
                              auto cnt_c) {
            constexpr int J0 = decltype(j0_c)::value, CNT = decltype(cnt_c)::value;
#pragma unroll
            for (int x = 0; x < STEP; ++x) {
                acc[x / MJ][x % MJ] = mfma_32x32x16<DT>(wf[x / MJ], af[x % MJ], acc[x / MJ][x % MJ]);
                const int from = x * CNT / STEP, to = (x + 1) * CNT / STEP;
                if (to > from) {
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int j = from; j < to; ++j) issue_one(tt, stage, J0 + j);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        using C0 = std::integral_constant<int, 0>;
        using CD0 = std::integral_constant<int, D0>;
        using CD1 = std::integral_constant<int, D1>;
        using CD2 = std::integral_constant<int, D2>;
        using CD01 = std::integral_constant<int, D0 + D1>;
        if (ktiles > 0) issue(0, 0);
        if (ktiles > 1) issue(1, 1);
        hold_epilogue_args();
        if (ktiles > 1) wait_vmcnt<IPW>();
        else wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        read_frags(ring, 0, af0, wf0);
        int cur = 0;   // ring stage of tile t
        // COPY: whether tile t + 2 exists (false for the last two tiles).
        // A wave issues its K-steps at raised priority (3, the highest) and
        // drops it before the wait for the next tile, so where waves share a
        // SIMD (8-wave workgroups, or several 64 x 64 workgroups per CU) one
        // whose neighbour already waits at its barrier keeps its MFMAs and
        // copies first in line: 2048 x 4096 x 1024 20.7 / 20.1 -> 19.2 /
        // 19.1 us in two runs (20.0 / 19.4 at priority 1), 4096^3 120.5 ->
        // 117.3 us, 64 x 64 tiles on 512 x 4096 x 1024 9.2 / 8.5 -> 8.5 /
        // 8.0 us and 2048 x 1024 x 2048 14.9 / 14.2 -> 14.1 / 13.6 us; no
        // change with one wave per SIMD.  (The 2-deep burst schedule below
        // raises it for its copies instead.)
        auto k_tile = [&](int t, auto copy_c) {
            constexpr bool COPY = decltype(copy_c)::value;
            const u32x4_t* tile = ring + cur * STAGE_CHUNKS;
            const int refill = cur == 0 ? STAGES - 1 : cur - 1;
            __builtin_amdgcn_s_setprio(3);
            read_frags(tile, 1, af1, wf1);
            if constexpr (COPY) mfmas_copy(af0, wf0, t + 2, refill, C0{}, CD0{});
            else mfmas(af0, wf0);
            read_frags(tile, 2, af0, wf0);
            if constexpr (COPY) mfmas_copy(af1, wf1, t + 2, refill, CD0{}, CD1{});
            else mfmas(af1, wf1);
            read_frags(tile, 3, af1, wf1);
            if constexpr (COPY) mfmas_copy(af0, wf0, t + 2, refill, CD01{}, CD2{});
            else mfmas(af0, wf0);
            const int next = cur + 1 == STAGES ? 0 : cur + 1;
            __builtin_amdgcn_s_setprio(0);
            if (t + 1 < ktiles) {
                if constexpr (COPY) wait_vmcnt<IPW>();
                else wait_vmcnt<0>();
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                read_frags(ring + next * STAGE_CHUNKS, 0, af0, wf0);
            }
            cur = next;
            mfmas(af1, wf1);
        };
        int t = 0;
        for (; t + 2 < ktiles; ++t) k_tile(t, std::true_type{});
        for (; t < ktiles; ++t) k_tile(t, std::false_type{});
    } else {
#pragma unroll
        for (int t = 0; t < AHEAD; ++t)
            if (t < ktiles) issue(t, t);
        hold_epilogue_args();
        tile_ready(0, STAGES - 1);
        read_frags(ring, 0, af0, wf0);

        int cur = 0;   // ring stage of tile t
        for (int t = 0; t < ktiles; ++t) {
            const u32x4_t* tile = ring + cur * STAGE_CHUNKS;
            read_frags(tile, 1, af1, wf1);
            mfmas(af0, wf0);
            read_frags(tile, 2, af0, wf0);
            mfmas(af1, wf1);
            read_frags(tile, 3, af1, wf1);
            mfmas(af0, wf0);
            const int next = cur + 1 == STAGES ? 0 : cur + 1;
            if (t + 1 < ktiles) {
                tile_ready(t + 1, cur);
                read_frags(ring + next * STAGE_CHUNKS, 0, af0, wf0);
            }
            cur = next;
            mfmas(af1, wf1);
        }
    }

    // Epilogue through LDS.  acc[i][j][v] is D[n][m] with n = 8 (v/4) +
    // 4 half + v%4 and m = l % 32 inside the (i, j) block, so each quad v/4
    // is 4 consecutive columns of one output row.  The quads are converted
    // and written into a BM x BN tile in LDS (row pitch padded by 16 bytes so
    // the 32 rows one store instruction touches spread over the banks), then
    // all the workgroup's threads copy the tile out row by row, 16 bytes per
    // lane, so every global store instruction writes whole row segments.
    // The copy-out stores are non-temporal: C is written once and not read
    // back by this launch, so it is kept out of L2 where it would evict the
    // A and W tiles other workgroups still read (2048 x 4096 x 1024 bf16:
    // 21.4 -> 19.6 us).
    constexpr int CPR = BNO * OB / 16;                           // 16-byte chunks per row
    static_assert(NT % CPR == 0, "rows per copy pass");
    char* ctile = reinterpret_cast<char*>(ring);
    if constexpr (EPASS > 1) {
        // Plain store of a C tile larger than LDS: one row of the wave grid
        // (EP_ROWS = WM rows) per pass, staged and copied out as below.
        constexpr int EPC = 16 / OB;
        constexpr int ROWS_PER_PASS = NT / CPR;
        static_assert(EP_ROWS % ROWS_PER_PASS == 0, "copy passes");
        const int chunk = tid % CPR;
        for (int ep = 0; ep < EPASS; ++ep) {
            __syncthreads();   // the K loop's last reads, or the previous pass's stores, are done with LDS
            if (wm == ep) {
#pragma unroll
                for (int j = 0; j < MJ; ++j) {
#pragma unroll
                    for (int i = 0; i < NI; ++i) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const f32x16_t& v = acc[i][j];
                            char* dst = ctile + (32 * j + r32) * PITCH + (wn * WN + 32 * i + 8 * q + 4 * half) * OB;
                            if constexpr (DT_OUT == NANOVLLM_GEMM_F32) {
                                *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                            } else {
                                *reinterpret_cast<u32x2_t*>(dst) =
                                    u32x2_t{pack2<DT_OUT>(v[4 * q], v[4 * q + 1]), pack2<DT_OUT>(v[4 * q + 2], v[4 * q + 3])};
                            }
                        }
                    }
                }
            }
            __syncthreads();
            const int64_t mp = m0 + int64_t(ep) * EP_ROWS;   // output row of C-tile row 0
            if (c_vec && mp + EP_ROWS <= m && n0 + BNO <= n) {
#pragma unroll
                for (int pass = 0; pass < EP_ROWS / ROWS_PER_PASS; ++pass) {
                    const int r = tid / CPR + pass * ROWS_PER_PASS;
                    const u32x4_t val = *reinterpret_cast<const u32x4_t*>(ctile + r * PITCH + chunk * 16);
                    __builtin_nontemporal_store(
                        val, reinterpret_cast<u32x4_t*>(static_cast<char*>(c) + ((mp + r) * ldc + n0 + chunk * EPC) * OB));
                }
                continue;
            }
            for (int r = tid / CPR; r < EP_ROWS; r += ROWS_PER_PASS) {
                const int64_t grow = mp + r;
                const int64_t gcol = n0 + chunk * EPC;
                if (grow >= m || gcol >= n) continue;
                const u32x4_t val = *reinterpret_cast<const u32x4_t*>(ctile + r * PITCH + chunk * 16);
                char* gdst = static_cast<char*>(c) + (grow * ldc + gcol) * OB;
                if (c_vec && gcol + EPC <= n) {
                    __builtin_nontemporal_store(val, reinterpret_cast<u32x4_t*>(gdst));
                } else {
                    const int valid = int(min_i64(EPC, n - gcol));
                    if constexpr (OB == 4) {
                        for (int e = 0; e < valid; ++e) reinterpret_cast<uint32_t*>(gdst)[e] = val[e];
                    } else {
                        for (int e = 0; e < valid; ++e)
                            reinterpret_cast<uint16_t*>(gdst)[e] = uint16_t(val[e >> 1] >> (16 * (e & 1)));
                    }
                }
            }
        }
        return;
    }
    __syncthreads();   // every wave is done reading the last K-tile
    constexpr int NIO = EPI == EPI_SILU_MUL ? NI / 2 : NI;     // 32-column output groups per wave
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int row = wm * WM + 32 * j + r32;
        float rs = 1.0f;
        if constexpr (RS) rs = row_scale[min_i64(m0 + row, m - 1)];
#pragma unroll
        for (int i = 0; i < NIO; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = wn * (NIO * 32) + 32 * i + 8 * q + 4 * half;
                float x0, x1, x2, x3;
                if constexpr (EPI == EPI_SILU_MUL) {
                    const f32x16_t& g = acc[2 * i][j];
                    const f32x16_t& u = acc[2 * i + 1][j];
                    if constexpr (RS) {
                        x0 = silu_f32(g[4 * q] * rs) * (u[4 * q] * rs);
                        x1 = silu_f32(g[4 * q + 1] * rs) * (u[4 * q + 1] * rs);
                        x2 = silu_f32(g[4 * q + 2] * rs) * (u[4 * q + 2] * rs);
                        x3 = silu_f32(g[4 * q + 3] * rs) * (u[4 * q + 3] * rs);
                    } else {
                        x0 = silu_f32(g[4 * q]) * u[4 * q];
                        x1 = silu_f32(g[4 * q + 1]) * u[4 * q + 1];
                        x2 = silu_f32(g[4 * q + 2]) * u[4 * q + 2];
                        x3 = silu_f32(g[4 * q + 3]) * u[4 * q + 3];
                    }
                } else {
                    const f32x16_t& v = acc[i][j];
                    x0 = v[4 * q]; x1 = v[4 * q + 1]; x2 = v[4 * q + 2]; x3 = v[4 * q + 3];
                    if constexpr (RS) {
                        x0 *= rs; x1 *= rs; x2 *= rs; x3 *= rs;
                    }
                }
                char* dst = ctile + row * PITCH + col * OB;
                if constexpr (DT_OUT == NANOVLLM_GEMM_F32) {
                    *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{x0, x1, x2, x3};
                } else {
                    *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{pack2<DT_OUT>(x0, x1), pack2<DT_OUT>(x2, x3)};
                }
            }
        }
    }
    __syncthreads();
    if constexpr (EPI == EPI_ARGMAX) {
        // Greedy LM head: per row of the tile, the best of its BN columns
        // (two threads per row, 64 columns each), one key per row.
        static_assert(OB == 4 && NT == 2 * BM, "fp32 tile, two threads per row");
        const int r = tid >> 1, h = tid & 1;
        const float* rowp = reinterpret_cast<const float*>(ctile + r * PITCH);
        uint64_t best = 0;
        if (m0 + r < m) {
            // Groups of 4 adjacent columns: one noise draw serves 4 scores on
            // a sampled row (n0 is a multiple of BN).
            const float t = sample_temperature(m0 + r, sa);
            for (int c4 = 0; c4 < BN / 2; c4 += 4) {
                const int col0 = h * (BN / 2) + c4;
                if (n0 + col0 >= n) break;
                const u32x4_t x = t != 0.0f ? sample_words(m0 + r, (n0 + col0) >> 2, sa) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = col0 + j;
                    if (n0 + col >= n) break;
                    const float v = ranked_logit(rowp[col], sa);
                    const uint64_t key = argmax_key(t != 0.0f ? gumbel_score(v, t, x[j]) : v, n0 + col);
                    best = key > best ? key : best;
                }
            }
        }
        const uint64_t other = (uint64_t(uint32_t(__shfl_xor(int(best >> 32), 1))) << 32) |
                               uint64_t(uint32_t(__shfl_xor(int(best & 0xFFFFFFFFu), 1)));
        best = other > best ? other : best;
        if (h == 0 && m0 + r < m) keys[(m0 + r) * int64_t(tiles_n) + tn] = best;
        return;
    }
    constexpr int EPC = 16 / OB;                 // output elements per chunk
    constexpr int ROWS_PER_PASS = NT / CPR;
    const int chunk = tid % CPR;
    if (c_vec && m0 + BM <= m && n0 + BNO <= n) {
        // Interior tile (uniform branch): whole 16-byte chunks, no masks.
        static_assert(BM % ROWS_PER_PASS == 0, "copy passes");
#pragma unroll
        for (int pass = 0; pass < BM / ROWS_PER_PASS; ++pass) {
            const int r = tid / CPR + pass * ROWS_PER_PASS;
            const u32x4_t val = *reinterpret_cast<const u32x4_t*>(ctile + r * PITCH + chunk * 16);
            __builtin_nontemporal_store(
                val, reinterpret_cast<u32x4_t*>(static_cast<char*>(c) + ((m0 + r) * ldc + n0 + chunk * EPC) * OB));
        }
        return;
    }
    for (int r = tid / CPR; r < BM; r += ROWS_PER_PASS) {
        const int64_t grow = m0 + r;
        const int64_t gcol = n0 + chunk * EPC;
        if (grow >= m || gcol >= n) continue;
        const u32x4_t val = *reinterpret_cast<const u32x4_t*>(ctile + r * PITCH + chunk * 16);
        char* gdst = static_cast<char*>(c) + (grow * ldc + gcol) * OB;
        if (c_vec && gcol + EPC <= n) {
            __builtin_nontemporal_store(val, reinterpret_cast<u32x4_t*>(gdst));
        } else {
            const int valid = int(min_i64(EPC, n - gcol));
            if constexpr (OB == 4) {
                for (int e = 0; e < valid; ++e) reinterpret_cast<uint32_t*>(gdst)[e] = val[e];
            } else {
                for (int e = 0; e < valid; ++e)
                    reinterpret_cast<uint16_t*>(gdst)[e] = uint16_t(val[e >> 1] >> (16 * (e & 1)));
            }
        }
    }
}

constexpr int64_t kCus = 256;

template <int DT, int DT_OUT, int BM, int BN, int WGM, int WGN, int STAGES, int EPI, int RS, int SP, int KN = 0>
int launch_tile(const Problem& p, hipStream_t s) {
    constexpr int BNO = EPI == EPI_SILU_MUL ? BN / 2 : BN;
    const int64_t tiles_m = (p.m + BM - 1) / BM, tiles_n = (p.n + BNO - 1) / BNO;
    if (tiles_m * tiles_n > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "mfma_staged: grid too large");
    if (p.k > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "mfma_staged: k must be below 2^31");
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n)), block(WGM * WGN * 64);
    const int out_bytes = DT_OUT == NANOVLLM_GEMM_F32 ? 4 : 2;
    // The copy-out writes 16-byte chunks: every row start must be 16-byte aligned.
    const int c_vec = (reinterpret_cast<uintptr_t>(p.c) % 16 == 0) && ((p.ldc * out_bytes) % 16 == 0);
    if (EPI == EPI_ARGMAX) *p.key_blocks = tiles_n;
    hipLaunchKernelGGL((mfma_staged_kernel<DT, DT_OUT, BM, BN, WGM, WGN, STAGES, EPI, RS, SP, KN>), grid, block, 0, s,
                       static_cast<const uint16_t*>(p.a), static_cast<const uint16_t*>(p.b), p.m, p.n, p.k, p.lda,
                       p.ldb, p.c, p.ldc, c_vec, p.keys, p.row_scale, p.sample);
    return check_launch("mfma_staged");
}

// Tile and schedule by grid size (bf16, MI355X, one launch; every choice
// sums K in the same order, so none changes a result bit).  "tiles" counts
// 128 x 128 tiles, "wide" 128 x 256 ones:
//   * tiles <= 128 (half the CUs): 64 x 64 tiles, four times the workgroups
//     (1024^3 11.7 -> 6.8 us, 512 x 4096 x 1024 12.3 -> 8.1 us,
//     2048 x 1024 x 2048 20.6 -> 13.8 us, 512 x 1024 x 3584 33.0 -> 17.0 us),
//     on a 3-deep ring with spread copies (against a 2-deep burst ring:
//     1024^3 6.85 -> 6.57 us, 512 x 4096 x 1024 8.49 -> 8.04, 256 x 6144 x
//     1024 8.03 -> 7.46, 2048 x 1024 x 2048 14.2 -> 14.0, 512 x 1024 x 3584
//     27.3 -> 17.2); SiLU pairs take 64 x 128, also with spread copies on
//     a 3-deep ring;
//   * 128 < wide <= 256 or wide > 384: one 8-wave workgroup per CU on
//     128 x 256 (half the A reads of two 128 x 128 tiles), 3-deep ring,
//     copies spread between the MFMAs.  Against the 2-deep 128 x 128 burst
//     schedule below: wide 144 (2304 x 2048 x 1024) 17.5 -> 14.7 us, 160
//     (2048 x 2560) 17.8 -> 15.5, 192 (2048 x 3072 x 2048) 32.8 -> 28.4,
//     224 (2048 x 3584) 19.8 -> 18.0, 256 (2048 x 4096) 20.3 -> 18.9, 416
//     (2048 x 6656) 35.9 -> 33.2, 512 (2048 x 8192) 38.5 -> 36.6, 2384
//     (2048 x 37984) 172 -> 162;
//   * 256 < wide <= 384 (one full round of 128 x 256 tiles and a partial
//     second): the 128 x 128 burst schedule with two workgroups per CU, whose
//     smaller tiles fill the second round better (wide 288 / 320 / 352 /
//     384: 29.1 / 30.1 / 29.4 / 30.4 us against 30.8 / 32.0 / 32.2 / 32.6);
//   * otherwise (128 < tiles <= 256): 128 x 128, 4 waves, 3-deep ring,
//     spread copies, one workgroup per CU (4096 x 1024 x 3584, 256 tiles:
//     40.0 -> 31.1 us against the burst schedule);
//   * the greedy head, whose epilogue is written for 4 waves, takes the
//     128 x 128 choices only;
//   * fp32 outputs (logits) over a W larger than the Infinity Cache, with at
//     least four rounds of 256 x 256 tiles and no more padded rows than
//     128-row tiles: 256 x 256 tiles (8 waves of 128 x 64, 2-deep ring,
//     burst copies; per flop two thirds of the bytes a 128 x 256 tile copies
//     into LDS, and half the passes over W).  Against 128 x 256, four
//     interleaved runs of each library in one process, bit-identical
//     outputs: 512 x 151936 x 1024 212.1-213.0 -> 202.1-207.3 us, 1024 x
//     151936 x 1024 404.0-405.0 -> 389.0-397.3 us; with a smaller W or bf16
//     outputs it measured the same (2048 x 37984 fp32 183.8-184.8 against
//     183.7-184.6, 512 x 151936 bf16 185.1-185.4 against 182.3-185.7, and
//     bf16 2048 x 37984, 2048 x 8192, 4096 x 4096, 4096 x 8192 within 1-2%).
//     On the LM head at M = 768 (seven rounds, both tile shapes ending on a
//     nearly full round) they tie, 300.4-301.5 against 299.1-299.7 us; at
//     M = 256 (2.3 rounds, below the threshold) 256 x 256 lost 4%.
constexpr int64_t kSmallGridTiles = kCus / 2;
constexpr int64_t kInfinityCacheBytes = int64_t(256) << 20;

// Whether an fp32-output plain GEMM takes 256 x 256 tiles (the rule above).
bool square256_tiles(const Problem& p) {
    const int64_t tiles_m128 = (p.m + 127) / 128;
    if (tiles_m128 % 2 != 0) return false;   // 256-row tiles would pad 128 more rows
    const int64_t tiles = tiles_m128 / 2 * ((p.n + 255) / 256);
    if (tiles < 4 * kCus) return false;
    return p.dtype_out == NANOVLLM_GEMM_F32 && p.n * p.k * 2 > kInfinityCacheBytes;
}

template <int DT, int DT_OUT, int EPI, int RS = 0>
int launch_epi(const Problem& p, hipStream_t s) {
    // A fused gate/up tile covers half its W rows in output columns.
    const int64_t n_tiles = EPI == EPI_SILU_MUL ? 2 * p.n : p.n;
    const int64_t tiles = ((p.m + 127) / 128) * ((n_tiles + 127) / 128);
    if (tiles <= kSmallGridTiles) {
        if constexpr (EPI == EPI_NONE) {
            return launch_tile<DT, DT_OUT, 64, 64, 2, 2, 3, EPI, RS, 1>(p, s);
        } else if constexpr (EPI == EPI_SILU_MUL) {
            // gate/up pairs need two 32-row W blocks per wave: 64 x 128
            // tiles, spread copies on a 3-deep ring (gate_up n = 3584, K =
            // 1024, M = 96 / 128 / 256: 9.4 / 9.4-9.7 / 9.6-10.5 -> 8.7 /
            // 8.6-8.9 / 8.8-9.4 us against the 2-deep burst ring, and
            // 15.7-17.0 -> 14.5-14.8 us at K = 2048 against the 3-deep one)
            return launch_tile<DT, DT_OUT, 64, 128, 2, 2, 3, EPI, RS, 1>(p, s);
        }
    }
    if constexpr (EPI == EPI_NONE && !RS && DT_OUT == NANOVLLM_GEMM_F32) {
        if (square256_tiles(p)) return launch_tile<DT, DT_OUT, 256, 256, 2, 4, 2, EPI, RS, 0>(p, s);
    }
    if constexpr (EPI != EPI_ARGMAX) {
        const int64_t wide = ((p.m + 127) / 128) * ((n_tiles + 255) / 256);
        if (wide > kCus / 2 && (wide <= kCus || wide > 3 * kCus / 2))
            return launch_tile<DT, DT_OUT, 128, 256, 2, 4, 3, EPI, RS, 1>(p, s);
    }
    if (tiles <= kCus) return launch_tile<DT, DT_OUT, 128, 128, 2, 2, 3, EPI, RS, 1>(p, s);
    return launch_tile<DT, DT_OUT, 128, 128, 2, 2, 2, EPI, RS, 0>(p, s);
}

// B[K,N]: the same tiles and copy schedules by grid size as W[N,K] (64 x 64
// up to 128 tiles of 128 x 128, 128 x 256 where those fill the CUs, 128 x
// 128 otherwise); the W part of each stage is B's k-rows as they lie in
// memory, read back with the transposing fragment read.
template <int DT, int DT_OUT>
int launch_kn(const Problem& p, hipStream_t s) {
    const int64_t tiles = ((p.m + 127) / 128) * ((p.n + 127) / 128);
    if (tiles <= kSmallGridTiles) return launch_tile<DT, DT_OUT, 64, 64, 2, 2, 3, EPI_NONE, 0, 1, 1>(p, s);
    const int64_t wide = ((p.m + 127) / 128) * ((p.n + 255) / 256);
    if (wide > kCus / 2 && (wide <= kCus || wide > 3 * kCus / 2))
        return launch_tile<DT, DT_OUT, 128, 256, 2, 4, 3, EPI_NONE, 0, 1, 1>(p, s);
    if (tiles <= kCus) return launch_tile<DT, DT_OUT, 128, 128, 2, 2, 3, EPI_NONE, 0, 1, 1>(p, s);
    return launch_tile<DT, DT_OUT, 128, 128, 2, 2, 2, EPI_NONE, 0, 0, 1>(p, s);
}

template <int DT, int DT_OUT>
int launch_typed(const Problem& p, hipStream_t s) {
    if (p.b_layout == NANOVLLM_GEMM_B_KN) {
        if (p.row_scale != nullptr || p.epi != EPI_NONE)
            return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "mfma_staged: B[K,N] takes the plain GEMM only");
        return launch_kn<DT, DT_OUT>(p, s);
    }
    if (p.row_scale != nullptr) {
        if (p.epi == EPI_SILU_MUL) return launch_epi<DT, DT_OUT, EPI_SILU_MUL, 1>(p, s);
        return launch_epi<DT, DT_OUT, EPI_NONE, 1>(p, s);
    }
    if (p.epi == EPI_SILU_MUL) return launch_epi<DT, DT_OUT, EPI_SILU_MUL>(p, s);
    return launch_epi<DT, DT_OUT, EPI_NONE>(p, s);
}

}  // namespace

int launch_mfma_staged(const Problem& p, hipStream_t s) {
    if (p.epi == EPI_ARGMAX) {
        constexpr int F = NANOVLLM_GEMM_F32;
        if (p.dtype_in == NANOVLLM_GEMM_BF16) return launch_epi<NANOVLLM_GEMM_BF16, F, EPI_ARGMAX>(p, s);
        return launch_epi<NANOVLLM_GEMM_F16, F, EPI_ARGMAX>(p, s);
    }
    if (p.dtype_in == NANOVLLM_GEMM_BF16) {
        if (p.dtype_out == NANOVLLM_GEMM_BF16) return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_BF16>(p, s);
        return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_F32>(p, s);
    }
    if (p.dtype_out == NANOVLLM_GEMM_F16) return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F16>(p, s);
    return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F32>(p, s);
}

}  // namespace nvg
