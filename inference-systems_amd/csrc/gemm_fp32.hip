// FP32 GEMM kernels for gfx950.
//
//   fp32_naive  — one thread per output, sequential K (the first rung of the
//                 reference ladder: cuda_kernels/gemm/src/gemm.cu:7-15,
//                 gemm_tiled.cu:36-51).
//   fp32_tiled  — 64x64 output tile per 512-thread workgroup, K-tiles of 64
//                 staged in LDS (one barrier per K-tile), products on the
//                 fp32 matrix cores with v_mfma_f32_32x32x2_f32 (full fp32
//                 precision; gfx950 has no reduced-precision fp32 MFMA).
//                 Replaces the shared-memory and register-tiled rungs
//                 (gemm_tiled.cu:56-202), including their zero-filled edge
//                 tiles, so any M, N, K and either B layout runs.  Problems
//                 whose rows are whole 16-byte chunks take fp32_staged_kernel
//                 (copies straight into a 3-deep LDS ring); the rest take
//                 fp32_tiled_kernel (scalar loads staged through registers
//                 into a double-buffered LDS tile).
#include <type_traits>

#include "gemm_common.hpp"

namespace nvg {
namespace {

template <int BL>
__global__ __launch_bounds__(256) void fp32_naive_kernel(
    const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int tiles_n) {
    const int tile = blockIdx.x;
    const int64_t row = int64_t(tile / tiles_n) * 16 + (threadIdx.x >> 4);
    const int64_t col = int64_t(tile % tiles_n) * 16 + (threadIdx.x & 15);
    if (row >= m || col >= n) return;
    const float* arow = a + row * lda;
    float sum = 0.0f;
    if constexpr (BL == NANOVLLM_GEMM_B_NK) {
        const float* wrow = b + col * ldb;
        for (int64_t kk = 0; kk < k; ++kk) sum = __builtin_fmaf(arow[kk], wrow[kk], sum);
    } else {
        for (int64_t kk = 0; kk < k; ++kk) sum = __builtin_fmaf(arow[kk], b[kk * ldb + col], sum);
    }
    c[row * ldc + col] = sum;
}

// Barrier for the LDS hand-off between K-tiles: this wave's LDS writes have
// completed, then all waves meet.  __syncthreads() would also wait for every
// outstanding global load (its release fence drains vmcnt), which would end
// the register prefetch at each K-tile.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

constexpr int kT32BM = 64;
constexpr int kT32BN = 64;
constexpr int kT32BK = 64;
constexpr int kT32Pitch = kT32BK + 4;   // 68 floats: 16-lane ds_read_b128 groups hit 64 distinct banks
constexpr int kT32Cpr = kT32BK / 4;     // 16-byte chunks per row of an A / W tile
constexpr int kT32Threads = 512;        // 8 waves: two groups of 4 (2 x 2 over the tile)
constexpr int kT32ScalarLoads = kT32BM * kT32BK / kT32Threads;   // 4-byte loads per operand per thread
static_assert(kT32BM == 64 && kT32BN == 64, "B[K,N] tiles are read as rows of 64 floats");

template <int BL>
__global__ __launch_bounds__(kT32Threads) void fp32_tiled_kernel(
    const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n) {
    // Both tiles are kept row-major over K ([row][k], pitch 68 floats), double
    // buffered.  For v_mfma_f32_32x32x2_f32 lane l supplies A(i = l%32, k) and
    // B(k, j = l%32) with the same k; MFMA step s of a K-tile uses
    // k = 16 (l/32) + s, so lane l needs 16 consecutive k of one row of each
    // tile and reads them with four ds_read_b128.
    //
    // Loads (8 scalar loads per operand per thread) are staged through two
    // register sets, two K-tiles ahead of the multiply (see `step` below).
    __shared__ __attribute__((aligned(16))) float As[2][kT32BM][kT32Pitch];
    __shared__ __attribute__((aligned(16))) float Bs[2][kT32BN][kT32Pitch];

    // K split inside the workgroup: wave group g (waves 4 g .. 4 g + 3, a
    // 2 x 2 grid of 32 x 32 blocks) multiplies K-half g of every K-tile into
    // its own accumulator, so each SIMD runs two waves whose LDS waits and
    // barrier stalls hide under the other's MFMAs; group 1 hands its
    // accumulator to group 0 through LDS at the end.
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int grp = wave >> 2;
    const int wm = (wave >> 1) & 1;
    const int wn = wave & 1;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int64_t m0 = int64_t(tm) * kT32BM;
    const int64_t n0 = int64_t(tn) * kT32BN;

    // Two register sets of staged loads, used by even and odd K-tiles.
    float ra[2][kT32ScalarLoads], rb[2][kT32ScalarLoads];

    // Every load is issued unconditionally from an address clamped into the
    // matrix; values outside the matrix are zeroed only when the tile is
    // written to LDS.  Straight-line loads whose results are not touched
    // until then keep the vmcnt bookkeeping exact and the loads in flight (a
    // branch around a load, or a select right after it, makes the compiler
    // wait for it at once).
    auto load_tile = [&](int64_t k0, auto set_c) {
        constexpr int S = decltype(set_c)::value;
#pragma unroll
        for (int r = 0; r < kT32ScalarLoads; ++r) {
            const int e = tid + kT32Threads * r;
            ra[S][r] = a[min_i64(m0 + e / kT32BK, m - 1) * lda + min_i64(k0 + e % kT32BK, k - 1)];
            if constexpr (BL == NANOVLLM_GEMM_B_NK)
                rb[S][r] = b[min_i64(n0 + e / kT32BK, n - 1) * ldb + min_i64(k0 + e % kT32BK, k - 1)];
            else
                rb[S][r] = b[min_i64(k0 + (e >> 6), k - 1) * ldb + min_i64(n0 + (e & 63), n - 1)];
        }
    };
    // Writes the K-tile starting at k0 (staged in register set S) to LDS
    // buffer `buf`, zeroing elements outside the matrix.
    auto store_tile = [&](int buf, int64_t k0, auto set_c) {
        constexpr int S = decltype(set_c)::value;
#pragma unroll
        for (int r = 0; r < kT32ScalarLoads; ++r) {
            const int e = tid + kT32Threads * r;
            const int row = e / kT32BK, kk = e % kT32BK;
            As[buf][row][kk] = (m0 + row < m && k0 + kk < k) ? ra[S][r] : 0.0f;
            if constexpr (BL == NANOVLLM_GEMM_B_NK)
                Bs[buf][row][kk] = (n0 + row < n && k0 + kk < k) ? rb[S][r] : 0.0f;
            else
                Bs[buf][e & 63][e >> 6] = (n0 + (e & 63) < n && k0 + (e >> 6) < k) ? rb[S][r] : 0.0f;
        }
    };

    using Set0 = std::integral_constant<int, 0>;
    using Set1 = std::integral_constant<int, 1>;
    f32x16_t acc = {};
    const int64_t ktiles = (k + kT32BK - 1) / kT32BK;
    // Prologue: K-tile 0 in LDS, K-tiles 1 (set 1) and 2 (set 0) in flight.
    load_tile(0, Set0{});
    store_tile(0, 0, Set0{});
    if (ktiles > 1) load_tile(kT32BK, Set1{});
    if (ktiles > 2) load_tile(2 * kT32BK, Set0{});
    lds_barrier();

    const int half = lane >> 5;
    const int ai = wm * 32 + (lane & 31);
    const int bj = wn * 32 + (lane & 31);
    // Each 32-wide K half of the tile is 16 MFMA steps; lane l takes k =
    // 32 h + 16 (l / 32) + s in step s of half h.  Group g takes half g.
    static_assert(kT32BK == 64, "one K half per wave group");
    auto multiply = [&](int buf) {
        {
            const int kh = grp;
            f32x4_t av[4], bv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                av[q] = *reinterpret_cast<const f32x4_t*>(&As[buf][ai][32 * kh + 16 * half + 4 * q]);
                bv[q] = *reinterpret_cast<const f32x4_t*>(&Bs[buf][bj][32 * kh + 16 * half + 4 * q]);
            }
#pragma unroll
            for (int st = 0; st < 16; ++st)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[st >> 2][st & 3], bv[st >> 2][st & 3], acc, 0, 0, 0);
        }
    };
    // K-tile t: register set (t + 1) % 2 holds K-tile t + 1 (loaded two
    // K-tiles ago); it goes to the free LDS buffer and is refilled with
    // K-tile t + 3, so every load has two K-tiles of MFMAs to arrive.  The
    // loop is unrolled by two so the set indices are compile-time constants.
    // The MFMAs run at raised wave priority (3), dropped before the
    // barrier: of the two waves on a SIMD, the one still multiplying issues
    // ahead of the one that has reached the barrier or its tile writes
    // (1024^3 B[K,N] 27.6 -> 26.7 us, 4096^3 1360 -> 1314 us).
    auto step = [&](int64_t t, auto set_c) {
        if (t + 1 < ktiles) store_tile(int((t + 1) & 1), (t + 1) * kT32BK, set_c);
        if (t + 3 < ktiles) load_tile((t + 3) * kT32BK, set_c);
        __builtin_amdgcn_s_setprio(3);
        multiply(int(t & 1));
        __builtin_amdgcn_s_setprio(0);
        lds_barrier();
    };
    for (int64_t t = 0; t < ktiles; t += 2) {
        step(t, Set1{});
        if (t + 1 < ktiles) step(t + 1, Set0{});
    }

    // Group 1's partial tile to group 0 through LDS (the last K-tile's
    // barrier has passed, so As is free): 16 values per lane.
    float* xch = &As[0][0][0];
    static_assert(4 * 16 * 64 <= 2 * kT32BM * kT32Pitch, "exchange fits in As");
    if (grp == 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) xch[((wave & 3) * 16 + v) * 64 + lane] = acc[v];
    }
    lds_barrier();
    if (grp == 1) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] += xch[((wave & 3) * 16 + v) * 64 + lane];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        const int64_t col = n0 + bj;
        if (row < m && col < n) __builtin_nontemporal_store(acc[v], c + row * ldc + col);
    }
}

// fp32_staged: the fp32_tiled rung for problems whose rows are whole 16-byte
// chunks (16-byte aligned bases and leading dimensions, K % 4 == 0, and N %
// 4 == 0 for B[K,N]).  Same 64 x 64 tile, same two K-groups of four waves
// and the same MFMA, but the operands move global -> LDS with
// global_load_lds_dwordx4 into a 3-deep ring, with no register staging and
// no LDS writes from the waves, and the copies of K-tile t + 2 are spread
// between the MFMAs of K-tile t.  Each wave reads its fragments a quarter
// K-tile ahead of its MFMAs and waits for the next K-tile before its last
// quarter, so the matrix cores stay busy across the one barrier per K-tile.
//
// LDS stage (32 KiB): the A tile (64 rows x 16 chunks of 4 k), then the B
// tile: W[N,K] rows like A; B[K,N] as 64 k-rows x 16 chunks of 4 columns,
// copied as they lie in memory and read back one float per lane.
//   A / W: chunk c of row r at position c ^ (r % 16): a ds_read_b128 of 16
//     consecutive rows at one chunk then touches 16 distinct positions, all
//     64 banks.
//   B[K,N]: chunk c of k-row r at position c ^ (8 ((r / 16) % 2)): the b32
//     read of one MFMA step takes 32 columns of k-rows r and r + 16, which
//     then sit in opposite halves of the banks.
constexpr int kF32StageChunks = 2 * kT32BM * kT32Cpr;   // 2048 16-byte chunks
constexpr int kF32Ipw = kF32StageChunks / (64 * (kT32Threads / 64));   // copies per wave per K-tile
static_assert(kF32Ipw == 4, "32 KiB per stage over 8 waves");
constexpr int kF32Stages = 3;   // ring depth (4 stages measured the same at 1024^3 and 2048^3)

// Source of the K-tail chunks: 16 zero bytes in global memory.
__device__ u32x4_t g_f32_zero = {0u, 0u, 0u, 0u};

template <int BL, int STAGES>
__global__ __launch_bounds__(kT32Threads) void fp32_staged_kernel(
    const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int tiles_m, int tiles_n) {
    constexpr int AHEAD = STAGES - 1;   // K-tiles in flight beyond the one multiplied
    static_assert(AHEAD >= 2 && AHEAD <= 3, "ring depth");
    __shared__ u32x4_t ring[STAGES * kF32StageChunks];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;
    const int wm = (wave >> 1) & 1;
    const int wn = wave & 1;
    const int half = lane >> 5;
    const int r32 = lane & 31;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int64_t m0 = int64_t(tm) * kT32BM;
    const int64_t n0 = int64_t(tn) * kT32BN;

    // Copy instruction j of this wave fills stage chunks 64 i .. 64 i + 63,
    // i = 4 wave + j: i < 16 rows 4 i .. 4 i + 3 of A, else rows (k-rows for
    // B[K,N]) 4 (i - 16) .. of B.  Lane L takes row 4 i' + L / 16, position
    // L % 16.  kpos[j]: the k (element of a row, or k-row of B[K,N]) its
    // chunk starts at within the K-tile.
    const float* src[kF32Ipw];
    int kpos[kF32Ipw];
    const int rin = lane >> 4, pos = lane & 15;
#pragma unroll
    for (int j = 0; j < kF32Ipw; ++j) {
        const int i = wave * kF32Ipw + j;
        if (i < 16) {
            const int row = 4 * i + rin;
            const int lc = pos ^ (row & 15);
            src[j] = a + min_i64(m0 + row, m - 1) * lda + 4 * lc;
            kpos[j] = 4 * lc;
        } else if constexpr (BL == NANOVLLM_GEMM_B_NK) {
            const int row = 4 * (i - 16) + rin;
            const int lc = pos ^ (row & 15);
            src[j] = b + min_i64(n0 + row, n - 1) * ldb + 4 * lc;
            kpos[j] = 4 * lc;
        } else {
            const int kr = 4 * (i - 16) + rin;
            const int lc = pos ^ (8 * ((kr >> 4) & 1));
            src[j] = b + int64_t(kr) * ldb + min_i64(n0 + 4 * lc, n - 4);
            kpos[j] = kr;
        }
    }
    const void* zero = &g_f32_zero;
    asm volatile("" : "+s"(zero));
    const int ktiles = static_cast<int>((k + kT32BK - 1) / kT32BK);
    const uint32_t ring_lds = lds_address(ring);
    auto issue_one = [&](int t, int stage, int j) {
        const int64_t k0 = int64_t(t) * kT32BK;
        const bool kn_row = BL == NANOVLLM_GEMM_B_KN && wave * kF32Ipw + j >= 16;
        const void* s = k0 + kpos[j] < k ? static_cast<const void*>(src[j] + (kn_row ? k0 * ldb : k0)) : zero;
        dma16(s, ring_lds + uint32_t(stage * kF32StageChunks + 64 * (wave * kF32Ipw + j)) * 16u);
    };
    auto issue = [&](int t, int stage) {
#pragma unroll
        for (int j = 0; j < kF32Ipw; ++j) issue_one(t, stage, j);
    };

    // Lane l takes k = 32 grp + 16 half + s of the K-tile in MFMA step s
    // (0..15); quarter q holds steps 4 q .. 4 q + 3, one 16-byte chunk of an
    // A (or W) row.
    const int ai = wm * 32 + r32;
    const int bj = wn * 32 + r32;
    struct Frag {
        f32x4_t a, b;
    };
    auto read_frag = [&](const u32x4_t* tile, int q) -> Frag {
        const int lc = 8 * grp + 4 * half + q;
        Frag f;
        f.a = __builtin_bit_cast(f32x4_t, tile[ai * kT32Cpr + (lc ^ (ai & 15))]);
        if constexpr (BL == NANOVLLM_GEMM_B_NK) {
            f.b = __builtin_bit_cast(f32x4_t, tile[kT32BM * kT32Cpr + bj * kT32Cpr + (lc ^ (bj & 15))]);
        } else {
            const float* bt = reinterpret_cast<const float*>(tile + kT32BM * kT32Cpr);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int kr = 4 * lc + s;
                f.b[s] = bt[(kr * kT32Cpr + ((bj >> 2) ^ (8 * ((kr >> 4) & 1)))) * 4 + (bj & 3)];
            }
        }
        return f;
    };
    f32x16_t acc = {};
    auto mfma4 = [&](const Frag& f) {
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[s], f.b[s], acc, 0, 0, 0);
    };
    // The 4 MFMAs of a quarter with copies J0 .. J0 + CNT - 1 of tile tt
    // after its first CNT MFMAs.
    auto mfma4_copy = [&](const Frag& f, int tt, int stage, int j0, int cnt) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[s], f.b[s], acc, 0, 0, 0);
            if (s < cnt) {
                __builtin_amdgcn_sched_barrier(0);
                issue_one(tt, stage, j0 + s);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // Tile u has landed in this wave's part of its stage once at most
    // `later` tiles issued after it are still in flight.
    auto wait_tiles_after = [&](int later) {
        if (AHEAD >= 3 && later >= 2) wait_vmcnt<2 * kF32Ipw>();
        else if (later >= 1) wait_vmcnt<kF32Ipw>();
        else wait_vmcnt<0>();
    };
#pragma unroll
    for (int u = 0; u < AHEAD; ++u)
        if (u < ktiles) issue(u, u);
    wait_tiles_after((ktiles < AHEAD ? ktiles : AHEAD) - 1);
    lds_barrier();
    Frag f0 = read_frag(ring, 0), f1;
    int cur = 0;
    // K-tile t: quarters 0-2 carry copies 2 / 1 / 1 of tile t + AHEAD into
    // the stage tile t - 1 used (free since the barrier that opened tile t);
    // the MFMAs run at raised wave priority, dropped before the wait for
    // tile t + 1.  COPY (whether tile t + AHEAD exists) is a compile-time
    // choice, and the tiles with and without copies run in two loops: a
    // branch between the two forms inside one loop body gives the
    // accumulator different registers on each path, and the copies that
    // join them wait for the MFMA chain.
    auto k_tile = [&](int t, auto copy_c) {
        constexpr bool COPY = decltype(copy_c)::value;
        const u32x4_t* tile = ring + cur * kF32StageChunks;
        const int refill = cur == 0 ? STAGES - 1 : cur - 1;
        const int next = cur + 1 == STAGES ? 0 : cur + 1;
        __builtin_amdgcn_s_setprio(3);
        f1 = read_frag(tile, 1);
        if constexpr (COPY) mfma4_copy(f0, t + AHEAD, refill, 0, 2);
        else mfma4(f0);
        f0 = read_frag(tile, 2);
        if constexpr (COPY) mfma4_copy(f1, t + AHEAD, refill, 2, 1);
        else mfma4(f1);
        f1 = read_frag(tile, 3);
        if constexpr (COPY) mfma4_copy(f0, t + AHEAD, refill, 3, 1);
        else mfma4(f0);
        __builtin_amdgcn_s_setprio(0);
        if (t + 1 < ktiles) {
            if constexpr (COPY) {
                if constexpr (AHEAD >= 3) wait_vmcnt<2 * kF32Ipw>();
                else wait_vmcnt<kF32Ipw>();
            } else {
                wait_tiles_after(ktiles - 2 - t);
            }
            lds_barrier();
            f0 = read_frag(ring + next * kF32StageChunks, 0);
        }
        cur = next;
        mfma4(f1);
    };
    int t = 0;
    for (; t + AHEAD < ktiles; ++t) k_tile(t, std::true_type{});
    for (; t < ktiles; ++t) k_tile(t, std::false_type{});

    // Group 1's partial tile to group 0 through LDS, once every wave is done
    // reading the last K-tile.
    lds_barrier();
    float* xch = reinterpret_cast<float*>(ring);
    if (grp == 1) {
#pragma unroll
        for (int v = 0; v < 16; ++v) xch[((wave & 3) * 16 + v) * 64 + lane] = acc[v];
    }
    lds_barrier();
    if (grp == 1) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] += xch[((wave & 3) * 16 + v) * 64 + lane];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        const int64_t col = n0 + bj;
        if (row < m && col < n) __builtin_nontemporal_store(acc[v], c + row * ldc + col);
    }
}

}  // namespace

int launch_fp32_naive(const Problem& p, hipStream_t s) {
    const int64_t tiles_m = (p.m + 15) / 16, tiles_n = (p.n + 15) / 16;
    if (tiles_m * tiles_n > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "fp32_naive: grid too large");
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n)), block(256);
    const float* a = static_cast<const float*>(p.a);
    const float* b = static_cast<const float*>(p.b);
    float* c = static_cast<float*>(p.c);
    if (p.b_layout == NANOVLLM_GEMM_B_NK)
        hipLaunchKernelGGL(fp32_naive_kernel<NANOVLLM_GEMM_B_NK>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                           p.lda, p.ldb, p.ldc, int(tiles_n));
    else
        hipLaunchKernelGGL(fp32_naive_kernel<NANOVLLM_GEMM_B_KN>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                           p.lda, p.ldb, p.ldc, int(tiles_n));
    return check_launch("fp32_naive");
}

int launch_fp32_tiled(const Problem& p, hipStream_t s) {
    const int64_t tiles_m = (p.m + kT32BM - 1) / kT32BM, tiles_n = (p.n + kT32BN - 1) / kT32BN;
    if (tiles_m * tiles_n > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "fp32_tiled: grid too large");
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n)), block(kT32Threads);
    const float* a = static_cast<const float*>(p.a);
    const float* b = static_cast<const float*>(p.b);
    float* c = static_cast<float*>(p.c);
    // The 16-byte copies of fp32_staged need aligned bases and leading dims
    // and chunks of 4 that do not straddle a row end: K % 4 == 0 (A and
    // W[N,K] rows), N % 4 == 0 (B[K,N] rows).
    const bool aligned = reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 &&
                         p.lda % 4 == 0 && p.ldb % 4 == 0 && p.k % 4 == 0;
    const bool staged = aligned && (p.b_layout == NANOVLLM_GEMM_B_NK || p.n % 4 == 0);
    const int ti = int(tiles_m), tj = int(tiles_n);
    if (p.b_layout == NANOVLLM_GEMM_B_NK) {
        if (staged)
            hipLaunchKernelGGL((fp32_staged_kernel<NANOVLLM_GEMM_B_NK, kF32Stages>), grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
        else
            hipLaunchKernelGGL(fp32_tiled_kernel<NANOVLLM_GEMM_B_NK>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
    } else {
        if (staged)
            hipLaunchKernelGGL((fp32_staged_kernel<NANOVLLM_GEMM_B_KN, kF32Stages>), grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
        else
            hipLaunchKernelGGL(fp32_tiled_kernel<NANOVLLM_GEMM_B_KN>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
    }
    return check_launch("fp32_tiled");
}

}  // namespace nvg
