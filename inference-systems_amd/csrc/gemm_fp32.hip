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
//                 whose rows are whole 16-byte chunks take fp32_buffered_kernel
//                 (buffer loads through registers into a double-buffered LDS
//                 tile, 32 x 32 or 64 x 64 tiles); the rest take
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

// fp32_buffered: the fp32_tiled rung for problems whose rows are whole
// 16-byte chunks (16-byte aligned bases and leading dimensions, K % 4 == 0,
// and N % 4 == 0 for B[K,N]).  A BM x BN tile per 4-wave workgroup (a 2 x 2
// grid of BM/2 x BN/2 wave tiles), K-tiles of BK:
//   * the operands are read with buffer loads into registers, one 16-byte
//     chunk per lane and instruction, and written to a double-buffered LDS
//     tile with ds_write_b128.  The buffer resources cover the tile's rows
//     (A, W[N,K]) or B[K,N]'s K rows, so rows past M / N and K-rows past K
//     read as zeros, and a chunk that starts at or past K is given an
//     out-of-range offset so it reads as zeros too;
//   * the loads of K-tile t + 3 are issued during K-tile t, into the register
//     set K-tile t + 1 has just left for the LDS, so every load has two
//     K-tiles of MFMAs to arrive (the loop is unrolled by two so both set
//     indices are compile-time constants);
//   * inside a K-tile the LDS writes of K-tile t + 1 ride on the first
//     MFMAs, the loads on the next, then one barrier, then the next K-tile's
//     fragments are read while the last quarter of this one's MFMAs runs;
//     the loop's back edge is at a point with no LDS access outstanding;
//   * LDS rows of A / W[N,K] hold chunk c of row r at c ^ swz(r) (16
//     consecutive rows at one chunk touch 16 distinct bank groups); B[K,N]
//     k-rows are copied as they lie, the column chunks of odd 16-k-row groups
//     flipped by half a row, so the two K halves of a wave's b32 reads sit
//     in opposite halves of the banks;
//   * MFMA step s of a K-tile takes k = STEPS (l / LH) + s in lane l, LH the
//     lanes per k group of the instruction, so a lane's A (and W[N,K])
//     values of a K-tile are one run of contiguous floats (ds_read_b128).
// Two configurations (measured on MI355X against the 8-wave copy-into-LDS
// kernel this replaces, in one process, fp32, B[K,N] unless noted):
//   * 64 x 32 tiles (wave tiles of 32 x 16: two 16 x 16 blocks, so two
//     independent v_mfma_f32_16x16x4_f32 chains per wave), BK = 64, while
//     the grid has fewer than 512 tiles of 64 x 64: two workgroups per CU
//     on 1024^3, so one's barrier waits hide under the other's MFMAs
//     (1024^3 21.7 -> 19.5 us; W[N,K] 21.5 -> 19.3 us);
//   * 64 x 64 tiles, v_mfma_f32_32x32x2_f32 in two accumulator chains (odd
//     steps in the second, added before the store), BK = 32, on larger grids
//     (2048^3 156.7 -> 126.6 us, 4096^3 1208.6 -> 966.6 us).
// Measured beside them: 64 x 64 tiles with one chain, BK = 32, 20.6 / 148.4
// / 959.6 us; 32 x 32 tiles, BK = 64, 19.2-20.8 / 143 / 1107 us; one
// K-tile of loads in flight more or less, half a K-tile of MFMAs after the
// barrier instead of a quarter, or capping the waves per SIMD at 2-4, moved
// 1024^3 by at most 1% (two waves per SIMD: 3% slower).  A v_mfma_f32_16x16x4_f32
// chain alone sustains 111 TFLOP/s at one wave per SIMD, two chains 150, and
// one v_mfma_f32_32x32x2_f32 chain 153 (157.3 peak).
// Chunk c of LDS row r of an A or W[N,K] tile sits at c ^ fp32_row_swizzle(r).
// The LDS serves a wave's ds_read_b128 in four groups of 16 lanes, lanes
// sharing bit 5 and the parity of bits 2-4 of the lane index (measured by
// the lane-map probe), and a fragment read puts lane l on row l % 16 (plus a
// multiple of 16), chunk 4 (l / 16) + q.  With 16 chunks per row the
// swizzle r ^ 8 bit2(r) gives the 16 lanes of each group 16 distinct
// chunks (plain r & 15 gives pairs the same chunk: 2-way conflicts on every
// fragment read); with 8 chunks per row (two rows per bank row) (r / 2) % 8
// does.  Both keep the 8 consecutive lanes of each ds_write_b128 clock on
// distinct chunks of one row.
__device__ __forceinline__ int fp32_row_swizzle(int r, int chunks) {
    return chunks == 16 ? ((r & 15) ^ (((r >> 2) & 1) << 3)) : ((r >> 1) & 7);
}

template <int BL, int BM, int BN, int BK, int MI, int CHN>
__global__ __launch_bounds__(256) void fp32_buffered_kernel(
    const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int tiles_m, int tiles_n) {
    constexpr int NT = 256;
    constexpr int WM = BM / 2, WN = BN / 2;             // wave tile
    constexpr int NBA = WM / MI, NBB = WN / MI;          // MI x MI blocks of the wave tile
    static_assert(NBA >= 1 && NBB >= 1 && WM % MI == 0 && WN % MI == 0, "wave tile");
    constexpr int ACH = BK / 4;                          // 16-byte chunks per row of a K-tile (A, W[N,K])
    constexpr int A_CH = BM * ACH;
    constexpr int KCH = BN / 4;                          // B[K,N]: chunks per k-row of a K-tile
    constexpr int STAGE = A_CH + BN * ACH;               // chunks per LDS stage
    constexpr int LPT = STAGE / NT;                      // loads per thread per K-tile
    constexpr int LA = A_CH / NT;                        // of which A
    static_assert(LPT * NT == STAGE && LA * NT == A_CH, "whole loads per thread");
    constexpr int STEPS = MI == 32 ? BK / 2 : BK / 4;    // MFMA K-steps per K-tile
    constexpr int LH = MI == 32 ? 32 : 16;               // lanes per k group of the MFMA
    __shared__ u32x4_t lds[2 * STAGE];
    auto kswz = [](int kr) { return (KCH / 2) * ((kr >> 4) & 1); };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
    // Byte ranges (the launcher checks they fit in 31 bits): the tile's rows
    // of A and W[N,K], all K rows of B[K,N] from column n0.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a + m0 * lda), short(0), int(((min_i64(BM, m - m0) - 1) * lda + k) * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        BL == NANOVLLM_GEMM_B_KN
            ? __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(b + n0), short(0), int(((k - 1) * ldb + (n - n0)) * 4),
                                                0x00020000)
            : __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(b + n0 * ldb), short(0),
                                                int(((min_i64(BN, n - n0) - 1) * ldb + k) * 4), 0x00020000);
    // Load j of a thread: chunk q = j NT + tid of the K-tile, A rows first.
    // voff: byte offset in its resource at K-tile 0; kpos: the k (A, W[N,K]
    // chunk) or k-row (B[K,N]) it starts at in the K-tile; dst: LDS chunk.
    uint32_t voff[LPT], dst[LPT];
    int kpos[LPT];
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
        const int q = (j < LA ? j : j - LA) * NT + tid;
        if (j < LA || BL == NANOVLLM_GEMM_B_NK) {
            const int r = q / ACH, ch = q % ACH;
            voff[j] = uint32_t((r * (j < LA ? lda : ldb) + ch * 4) * 4);
            dst[j] = uint32_t((j < LA ? 0 : A_CH) + r * ACH + (ch ^ fp32_row_swizzle(r, ACH)));
            kpos[j] = 4 * ch;
        } else {
            const int kr = q / KCH, ch = q % KCH;
            voff[j] = uint32_t((kr * ldb + ch * 4) * 4);
            dst[j] = uint32_t(A_CH + kr * KCH + (ch ^ kswz(kr)));
            kpos[j] = kr;
        }
    }
    const int ktiles = static_cast<int>((k + BK - 1) / BK);
    // Loads of K-tile t.  Before the last K-tile every chunk lies inside K
    // and inside the allocation, and the K-tile's offset goes in the scalar
    // offset.  The last K-tile (CHECKED) puts the whole offset in the lane's
    // offset register, which the range check covers, and gives chunks that
    // start at or past K an out-of-range offset, so they read as zeros.
    auto load_one = [&](u32x4_t& r, int j, int t, auto checked_c) {
        const int k0 = t * BK;
        const bool kn_row = BL == NANOVLLM_GEMM_B_KN && j >= LA;
        const uint32_t step = kn_row ? uint32_t(k0) * uint32_t(ldb) * 4u : uint32_t(k0) * 4u;
        if constexpr (decltype(checked_c)::value) {
            const uint32_t vo = k0 + kpos[j] < k ? voff[j] + step : 0x80000000u;
            r = __builtin_amdgcn_raw_buffer_load_b128(j < LA ? ra : rb, vo, 0, 0);
        } else {
            r = __builtin_amdgcn_raw_buffer_load_b128(j < LA ? ra : rb, voff[j], int(step), 0);
        }
    };
    using Checked = std::true_type;
    using Unchecked = std::false_type;
    u32x4_t rs[2][LPT];

    const int frow = lane % LH, fh = lane / LH;
    struct Frag { f32x4_t q[STEPS / 4]; };   // a lane's STEPS values of one block
    Frag fa0[NBA], fb0[NBB], fa1[NBA], fb1[NBB];
    auto read_frags = [&](int st, Frag (&fa)[NBA], Frag (&fb)[NBB]) {
        const u32x4_t* tile = lds + st * STAGE;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NBA; ++i) {
            const int r = wm * WM + MI * i + frow;
#pragma unroll
            for (int q = 0; q < STEPS / 4; ++q) {
                const int ch = (STEPS / 4) * fh + q;
                fa[i].q[q] = __builtin_bit_cast(f32x4_t, tile[r * ACH + (ch ^ fp32_row_swizzle(r, ACH))]);
            }
        }
#pragma unroll
        for (int i = 0; i < NBB; ++i) {
            const int col = wn * WN + MI * i + frow;
            if constexpr (BL == NANOVLLM_GEMM_B_KN) {
                const float* bt = reinterpret_cast<const float*>(tile + A_CH);
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    const int kr = STEPS * fh + s;
                    fb[i].q[s / 4][s % 4] = bt[kr * BN + (((col >> 2) ^ kswz(kr)) << 2) + (col & 3)];
                }
            } else {
#pragma unroll
                for (int q = 0; q < STEPS / 4; ++q) {
                    const int ch = (STEPS / 4) * fh + q;
                    fb[i].q[q] = __builtin_bit_cast(f32x4_t, tile[A_CH + col * ACH + (ch ^ fp32_row_swizzle(col, ACH))]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    typedef std::conditional_t<MI == 32, f32x16_t, f32x4_t> acc_t;
    acc_t acc[CHN][NBB][NBA];
#pragma unroll
    for (int h = 0; h < CHN; ++h)
#pragma unroll
        for (int i = 0; i < NBB; ++i)
#pragma unroll
            for (int j = 0; j < NBA; ++j) acc[h][i][j] = acc_t{};
    // The MFMAs of steps [S0, S1) with CNT of the memory operations `fn`
    // spread evenly between them (the scheduling barriers pin each one).
    auto mfmas = [&](const Frag (&fa)[NBA], const Frag (&fb)[NBB], auto s0_c, auto s1_c, auto fn, auto cnt_c) {
        constexpr int S0 = decltype(s0_c)::value, S1 = decltype(s1_c)::value, CNT = decltype(cnt_c)::value;
        constexpr int PER = NBA * NBB, TOT = (S1 - S0) * PER;
#pragma unroll
        for (int x = 0; x < TOT; ++x) {
            const int s = S0 + x / PER, i = (x / NBA) % NBB, j = x % NBA;
            acc_t& d = acc[s % CHN][i][j];
            // B's block (output columns) first: its rows are the rows of the product.
            if constexpr (MI == 32)
                d = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[i].q[s / 4][s % 4], fa[j].q[s / 4][s % 4], d, 0, 0, 0);
            else
                d = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[i].q[s / 4][s % 4], fa[j].q[s / 4][s % 4], d, 0, 0, 0);
            const int from = x * CNT / TOT, to = (x + 1) * CNT / TOT;
            if (to > from) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int y = from; y < to; ++y) fn(y);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    auto none = [](int) {};
    using C0 = std::integral_constant<int, 0>;
    using CL = std::integral_constant<int, LPT>;
    using SMID = std::integral_constant<int, (STEPS - STEPS / 4) / 2>;
    using STAIL = std::integral_constant<int, STEPS - STEPS / 4>;
    using SEND = std::integral_constant<int, STEPS>;

    // Prologue: K-tiles 0 and 1 into the register sets, K-tile 0 into stage
    // 0, K-tile 2 into set 0.
#pragma unroll
    for (int j = 0; j < LPT; ++j) load_one(rs[0][j], j, 0, Checked{});
    if (ktiles > 1) {
#pragma unroll
        for (int j = 0; j < LPT; ++j) load_one(rs[1][j], j, 1, Checked{});
    }
#pragma unroll
    for (int j = 0; j < LPT; ++j) lds[dst[j]] = rs[0][j];
    if (ktiles > 2) {
#pragma unroll
        for (int j = 0; j < LPT; ++j) load_one(rs[0][j], j, 2, Checked{});
    }
    lds_barrier();
    read_frags(0, fa0, fb0);
    // K-tile t, fragments in (fac, fbc): K-tile t + 1 from set SET into stage
    // (t + 1) % 2 (when it exists), then K-tile t + 3 into SET (when it
    // exists); the next K-tile's fragments go to (fan, fbn).
    auto k_tile = [&](int t, auto set_c, Frag (&fac)[NBA], Frag (&fbc)[NBB], Frag (&fan)[NBA], Frag (&fbn)[NBB],
                      bool load, bool write, auto checked_c) {
        constexpr int SET = decltype(set_c)::value;
        const int st = t & 1;
        auto ld = [&](int j) { load_one(rs[SET][j], j, t + 3, checked_c); };
        auto wr = [&](int j) { lds[(st ^ 1) * STAGE + dst[j]] = rs[SET][j]; };
        // The MFMAs before the barrier run at raised wave priority, dropped
        // before it: of the waves on a SIMD, those still multiplying issue
        // ahead of those that have reached the barrier.
        __builtin_amdgcn_s_setprio(3);
        if (write) mfmas(fac, fbc, C0{}, SMID{}, wr, CL{});
        else mfmas(fac, fbc, C0{}, SMID{}, none, C0{});
        if (load) mfmas(fac, fbc, SMID{}, STAIL{}, ld, CL{});
        else mfmas(fac, fbc, SMID{}, STAIL{}, none, C0{});
        __builtin_amdgcn_s_setprio(0);
        if (write) {
            lds_barrier();
            read_frags(st ^ 1, fan, fbn);
        }
        mfmas(fac, fbc, STAIL{}, SEND{}, none, C0{});
    };
    using Set0 = std::integral_constant<int, 0>;
    using Set1 = std::integral_constant<int, 1>;
    int t = 0;
    // Two K-tiles per trip; every load and write of the trip exists, and the
    // loads (of K-tiles t + 3, t + 4) precede the last K-tile.
    for (; t + 5 < ktiles; t += 2) {
        k_tile(t, Set1{}, fa0, fb0, fa1, fb1, true, true, Unchecked{});
        k_tile(t + 1, Set0{}, fa1, fb1, fa0, fb0, true, true, Unchecked{});
    }
    // The last (at most five) K-tiles as fixed sequences: t is even, so
    // K-tile t + i uses set (i + 1) % 2 and fragment set i % 2; the only load
    // into the last K-tile is the checked one.
    auto tail = [&](int i, auto load_c, auto write_c, auto checked_c) {
        constexpr bool LOAD = decltype(load_c)::value, WRITE = decltype(write_c)::value;
        if (i % 2 == 0) k_tile(t + i, Set1{}, fa0, fb0, fa1, fb1, LOAD, WRITE, checked_c);
        else k_tile(t + i, Set0{}, fa1, fb1, fa0, fb0, LOAD, WRITE, checked_c);
    };
    using T = std::true_type;
    using F = std::false_type;
    switch (ktiles - t) {
        case 5:
            tail(0, T{}, T{}, Unchecked{});
            tail(1, T{}, T{}, Checked{});
            tail(2, F{}, T{}, Unchecked{});
            tail(3, F{}, T{}, Unchecked{});
            tail(4, F{}, F{}, Unchecked{});
            break;
        case 4:
            tail(0, T{}, T{}, Checked{});
            tail(1, F{}, T{}, Unchecked{});
            tail(2, F{}, T{}, Unchecked{});
            tail(3, F{}, F{}, Unchecked{});
            break;
        case 3:
            tail(0, F{}, T{}, Unchecked{});
            tail(1, F{}, T{}, Unchecked{});
            tail(2, F{}, F{}, Unchecked{});
            break;
        case 2:
            tail(0, F{}, T{}, Unchecked{});
            tail(1, F{}, F{}, Unchecked{});
            break;
        default:
            tail(0, F{}, F{}, Unchecked{});
            break;
    }
    if constexpr (CHN == 2) {
#pragma unroll
        for (int i = 0; i < NBB; ++i)
#pragma unroll
            for (int j = 0; j < NBA; ++j) acc[0][i][j] += acc[1][i][j];
    }
    // acc[0][i][j][v]: MI = 32: D[n = 8 (v / 4) + 4 (l / 32) + v % 4][m = l % 32];
    // MI = 16: D[n = 4 (l / 16) + v][m = l % 16] of block (i, j): 4 adjacent
    // output columns of one row per quad.
#pragma unroll
    for (int i = 0; i < NBB; ++i)
#pragma unroll
        for (int j = 0; j < NBA; ++j) {
            const int64_t row = m0 + wm * WM + MI * j + frow;
#pragma unroll
            for (int q = 0; q < MI * MI / 256; ++q) {
                const int64_t col = n0 + wn * WN + MI * i + (MI == 32 ? 8 * q + 4 * fh : 4 * fh);
                const acc_t& v = acc[0][i][j];
                const f32x4_t o = f32x4_t{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                if (row >= m) continue;
                if (col + 3 < n && ldc % 4 == 0) {
                    __builtin_nontemporal_store(o, reinterpret_cast<f32x4_t*>(c + row * ldc + col));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < n) c[row * ldc + col + e] = o[e];
                }
            }
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

namespace {

template <int BL, int BM, int BN, int BK, int MI, int CHN>
void launch_buffered(const Problem& p, hipStream_t s) {
    const int64_t tiles_m = (p.m + BM - 1) / BM, tiles_n = (p.n + BN - 1) / BN;
    hipLaunchKernelGGL((fp32_buffered_kernel<BL, BM, BN, BK, MI, CHN>), dim3(static_cast<uint32_t>(tiles_m * tiles_n)),
                       dim3(256), 0, s, static_cast<const float*>(p.a), static_cast<const float*>(p.b),
                       static_cast<float*>(p.c), p.m, p.n, p.k, p.lda, p.ldb, p.ldc, int(tiles_m), int(tiles_n));
}

template <int BL>
void launch_buffered_for(const Problem& p, hipStream_t s) {
    const int64_t tiles64 = ((p.m + 63) / 64) * ((p.n + 63) / 64);
    if (tiles64 < 512) launch_buffered<BL, 64, 32, 64, 16, 1>(p, s);
    else launch_buffered<BL, 64, 64, 32, 32, 2>(p, s);
}

}  // namespace

int launch_fp32_tiled(const Problem& p, hipStream_t s) {
    const int64_t tiles_m = (p.m + kT32BM - 1) / kT32BM, tiles_n = (p.n + kT32BN - 1) / kT32BN;
    if (tiles_m * tiles_n > INT32_MAX / 4) return set_error(NANOVLLM_GEMM_EINVAL, "fp32_tiled: grid too large");
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n)), block(kT32Threads);
    const float* a = static_cast<const float*>(p.a);
    const float* b = static_cast<const float*>(p.b);
    float* c = static_cast<float*>(p.c);
    // The 16-byte loads of fp32_buffered need aligned bases and leading dims
    // and chunks of 4 that do not straddle a row end: K % 4 == 0 (A and
    // W[N,K] rows), N % 4 == 0 (B[K,N] rows); its buffer ranges are 31-bit
    // byte counts: 64 rows of A or W[N,K], or all of B[K,N] from a column.
    constexpr int64_t kRange = int64_t(1) << 31;
    const bool aligned = reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 &&
                         p.lda % 4 == 0 && p.ldb % 4 == 0 && p.k % 4 == 0;
    const bool ranges = 64 * p.lda * 4 < kRange &&
                        (p.b_layout == NANOVLLM_GEMM_B_NK ? 64 * p.ldb * 4 < kRange : p.k * p.ldb * 4 < kRange);
    const bool buffered = aligned && ranges && (p.b_layout == NANOVLLM_GEMM_B_NK || p.n % 4 == 0);
    const int ti = int(tiles_m), tj = int(tiles_n);
    if (p.b_layout == NANOVLLM_GEMM_B_NK) {
        if (buffered)
            launch_buffered_for<NANOVLLM_GEMM_B_NK>(p, s);
        else
            hipLaunchKernelGGL(fp32_tiled_kernel<NANOVLLM_GEMM_B_NK>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
    } else {
        if (buffered)
            launch_buffered_for<NANOVLLM_GEMM_B_KN>(p, s);
        else
            hipLaunchKernelGGL(fp32_tiled_kernel<NANOVLLM_GEMM_B_KN>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
    }
    return check_launch("fp32_tiled");
}

}  // namespace nvg
