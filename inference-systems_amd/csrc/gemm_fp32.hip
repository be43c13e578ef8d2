// FP32 GEMM kernels for gfx950.
//
//   fp32_naive  — one thread per output, sequential K (the first rung of the
//                 reference ladder: cuda_kernels/gemm/src/gemm.cu:7-15,
//                 gemm_tiled.cu:36-51).
//   fp32_tiled  — 64x64 output tile per 512-thread workgroup, K-tiles of 64
//                 staged in LDS (double buffered, one barrier per K-tile,
//                 fragments read with ds_read_b128 in a K-permuted order),
//                 products on the fp32 matrix cores with
//                 v_mfma_f32_32x32x2_f32 (full fp32 precision; gfx950 has no
//                 reduced-precision fp32 MFMA).  Replaces the shared-memory and
//                 register-tiled rungs (gemm_tiled.cu:56-202), including their
//                 zero-filled edge tiles, so any M, N, K and either B layout
//                 runs.
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
constexpr int kT32VecLoads = kT32BM * kT32Cpr / kT32Threads;     // 16-byte loads per operand per thread
constexpr int kT32ScalarLoads = kT32BM * kT32BK / kT32Threads;   // 4-byte loads per operand per thread
static_assert(kT32BM == 64 && kT32BN == 64, "B[K,N] tiles are read as rows of 64 floats");
static_assert(kT32VecLoads == 2 && kT32Threads == 512, "B[K,N]: one 2 x 4 block of the 64 x 64 tile per thread");
typedef float f32x2_t __attribute__((ext_vector_type(2)));

template <int BL, int VEC>
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
    // Loads are staged through two register sets, two K-tiles ahead of the
    // multiply (see `step` below).  VEC: 16-byte loads (2 per operand per
    // thread; needs 16-byte aligned rows), else 8 scalar loads per operand
    // per thread.
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
    f32x4_t va[2][VEC ? kT32VecLoads : 1], vb[2][VEC ? kT32VecLoads : 1];
    float ra[2][VEC ? 1 : kT32ScalarLoads], rb[2][VEC ? 1 : kT32ScalarLoads];

    // Every load is issued unconditionally from an address clamped into the
    // matrix; values outside the matrix are zeroed only when the tile is
    // written to LDS.  Straight-line loads whose results are not touched
    // until then keep the vmcnt bookkeeping exact and the loads in flight (a
    // branch around a load, or a select right after it, makes the compiler
    // wait for it at once).
    auto load_tile = [&](int64_t k0, auto set_c) {
        constexpr int S = decltype(set_c)::value;
        if constexpr (VEC) {
#pragma unroll
            for (int r = 0; r < kT32VecLoads; ++r) {
                const int e = tid + kT32Threads * r;     // 16-byte chunks of the operand tile
                const int64_t gm = m0 + e / kT32Cpr, gka = k0 + 4 * (e % kT32Cpr);   // A: chunks of 4 k per row
                va[S][r] = *reinterpret_cast<const f32x4_t*>(a + min_i64(gm, m - 1) * lda + min_i64(gka, k - 4));
                if constexpr (BL == NANOVLLM_GEMM_B_NK) {
                    const int64_t gn = n0 + e / kT32Cpr, gk = k0 + 4 * (e % kT32Cpr);
                    vb[S][r] = *reinterpret_cast<const f32x4_t*>(b + min_i64(gn, n - 1) * ldb + min_i64(gk, k - 4));
                } else {
                    // B[K,N]: thread t takes 4 columns (t % 16) of rows 2 (t / 16) and 2 (t / 16) + 1.
                    const int64_t gn = n0 + 4 * (tid & 15), gk = k0 + 2 * (tid >> 4) + r;
                    vb[S][r] = *reinterpret_cast<const f32x4_t*>(b + min_i64(gk, k - 1) * ldb + min_i64(gn, n - 4));
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < kT32ScalarLoads; ++r) {
                const int e = tid + kT32Threads * r;
                ra[S][r] = a[min_i64(m0 + e / kT32BK, m - 1) * lda + min_i64(k0 + e % kT32BK, k - 1)];
                if constexpr (BL == NANOVLLM_GEMM_B_NK)
                    rb[S][r] = b[min_i64(n0 + e / kT32BK, n - 1) * ldb + min_i64(k0 + e % kT32BK, k - 1)];
                else
                    rb[S][r] = b[min_i64(k0 + (e >> 6), k - 1) * ldb + min_i64(n0 + (e & 63), n - 1)];
            }
        }
    };
    // Writes the K-tile starting at k0 (staged in register set S) to LDS
    // buffer `buf`, zeroing elements outside the matrix.
    auto store_tile = [&](int buf, int64_t k0, auto set_c) {
        constexpr int S = decltype(set_c)::value;
        const f32x4_t z4 = {0.f, 0.f, 0.f, 0.f};
        if constexpr (VEC) {
#pragma unroll
            for (int r = 0; r < kT32VecLoads; ++r) {
                const int e = tid + kT32Threads * r;
                const int row = e / kT32Cpr, kq = e % kT32Cpr;
                const bool in_a = m0 + row < m && k0 + 4 * kq < k;
                *reinterpret_cast<f32x4_t*>(&As[buf][row][4 * kq]) = in_a ? va[S][r] : z4;
                if constexpr (BL == NANOVLLM_GEMM_B_NK) {
                    const bool in_b = n0 + row < n && k0 + 4 * kq < k;
                    *reinterpret_cast<f32x4_t*>(&Bs[buf][row][4 * kq]) = in_b ? vb[S][r] : z4;
                } else if (r == 1) {
                    // The thread's 2 x 4 block of B[K,N], transposed into 4
                    // pairs of consecutive k (one 8-byte write each).
                    const int nq = tid & 15, kp = tid >> 4;
                    const bool in_n = n0 + 4 * nq < n;
                    const bool in0 = in_n && k0 + 2 * kp < k, in1 = in_n && k0 + 2 * kp + 1 < k;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *reinterpret_cast<f32x2_t*>(&Bs[buf][4 * nq + q][2 * kp]) =
                            f32x2_t{in0 ? vb[S][0][q] : 0.0f, in1 ? vb[S][1][q] : 0.0f};
                }
            }
        } else {
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
    // 16-byte loads need aligned bases and leading dims (and, for A and W,
    // K-chunks of 4 that do not straddle K: K % 4 == 0; for B[K,N], N % 4).
    const bool aligned = reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 &&
                         p.lda % 4 == 0 && p.ldb % 4 == 0 && p.k % 4 == 0;
    const bool vec = aligned && (p.b_layout == NANOVLLM_GEMM_B_NK || p.n % 4 == 0);
    const int ti = int(tiles_m), tj = int(tiles_n);
    if (p.b_layout == NANOVLLM_GEMM_B_NK) {
        if (vec)
            hipLaunchKernelGGL((fp32_tiled_kernel<NANOVLLM_GEMM_B_NK, 1>), grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
        else
            hipLaunchKernelGGL((fp32_tiled_kernel<NANOVLLM_GEMM_B_NK, 0>), grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
    } else {
        if (vec)
            hipLaunchKernelGGL((fp32_tiled_kernel<NANOVLLM_GEMM_B_KN, 1>), grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
        else
            hipLaunchKernelGGL((fp32_tiled_kernel<NANOVLLM_GEMM_B_KN, 0>), grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                               p.lda, p.ldb, p.ldc, ti, tj);
    }
    return check_launch("fp32_tiled");
}

}  // namespace nvg
