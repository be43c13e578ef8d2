// FP32 GEMM kernels for gfx950.
//
//   fp32_naive  — one thread per output, sequential K (the first rung of the
//                 reference ladder: cuda_kernels/gemm/src/gemm.cu:7-15,
//                 gemm_tiled.cu:36-51).
//   fp32_tiled  — 64x64 output tile per 256-thread workgroup, K-tiles of 32
//                 staged in LDS (double buffered, one barrier per K-tile,
//                 fragments read with ds_read_b128 in a K-permuted order),
//                 products on the fp32 matrix cores with
//                 v_mfma_f32_32x32x2_f32 (full fp32 precision; gfx950 has no
//                 reduced-precision fp32 MFMA).  Replaces the shared-memory and
//                 register-tiled rungs (gemm_tiled.cu:56-202), including their
//                 zero-filled edge tiles, so any M, N, K and either B layout
//                 runs.
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

constexpr int kT32BM = 64;
constexpr int kT32BN = 64;
constexpr int kT32BK = 32;
constexpr int kT32Pitch = kT32BK + 4;   // 36 floats: 16-lane ds_read_b128 groups hit 64 distinct banks

template <int BL>
__global__ __launch_bounds__(256) void fp32_tiled_kernel(
    const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n) {
    // Both tiles are kept row-major over K ([row][k], pitch 36 floats), double
    // buffered.  For v_mfma_f32_32x32x2_f32 lane l supplies A(i = l%32, k) and
    // B(k, j = l%32) with the same k; MFMA step s of a K-tile uses
    // k = 16 (l/32) + s, so lane l needs 16 consecutive k of one row of each
    // tile and reads them with four ds_read_b128.
    __shared__ __attribute__((aligned(16))) float As[2][kT32BM][kT32Pitch];
    __shared__ __attribute__((aligned(16))) float Bs[2][kT32BN][kT32Pitch];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int64_t m0 = int64_t(tm) * kT32BM;
    const int64_t n0 = int64_t(tn) * kT32BN;

    float ra[8], rb[8];

    // Each thread moves 8 elements of each operand per K-tile.  A (and W in
    // the NK layout) is read along K: 32 consecutive threads cover one
    // 128-byte row segment.  B in the KN layout is read along N and written
    // transposed.
    auto load_tile = [&](int64_t k0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int e = tid + 256 * r;
            {
                const int row = e >> 5, kk = e & 31;
                const int64_t gm = m0 + row, gk = k0 + kk;
                ra[r] = (gm < m && gk < k) ? a[gm * lda + gk] : 0.0f;
            }
            if constexpr (BL == NANOVLLM_GEMM_B_NK) {
                const int col = e >> 5, kk = e & 31;
                const int64_t gn = n0 + col, gk = k0 + kk;
                rb[r] = (gn < n && gk < k) ? b[gn * ldb + gk] : 0.0f;
            } else {
                const int kk = e >> 6, col = e & 63;
                const int64_t gn = n0 + col, gk = k0 + kk;
                rb[r] = (gn < n && gk < k) ? b[gk * ldb + gn] : 0.0f;
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int e = tid + 256 * r;
            As[buf][e >> 5][e & 31] = ra[r];
            if constexpr (BL == NANOVLLM_GEMM_B_NK) {
                Bs[buf][e >> 5][e & 31] = rb[r];
            } else {
                Bs[buf][e & 63][e >> 6] = rb[r];
            }
        }
    };

    f32x16_t acc = {};
    const int64_t ktiles = (k + kT32BK - 1) / kT32BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();

    const int half = lane >> 5;
    const int ai = wm * 32 + (lane & 31);
    const int bj = wn * 32 + (lane & 31);
    for (int64_t t = 0; t < ktiles; ++t) {
        const int cur = int(t & 1);
        const bool more = t + 1 < ktiles;
        if (more) load_tile((t + 1) * kT32BK);
        f32x4_t av[4], bv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            av[q] = *reinterpret_cast<const f32x4_t*>(&As[cur][ai][16 * half + 4 * q]);
            bv[q] = *reinterpret_cast<const f32x4_t*>(&Bs[cur][bj][16 * half + 4 * q]);
        }
#pragma unroll
        for (int st = 0; st < kT32BK / 2; ++st)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[st >> 2][st & 3], bv[st >> 2][st & 3], acc, 0, 0, 0);
        if (more) store_tile(cur ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        const int64_t col = n0 + bj;
        if (row < m && col < n) c[row * ldc + col] = acc[v];
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
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n)), block(256);
    const float* a = static_cast<const float*>(p.a);
    const float* b = static_cast<const float*>(p.b);
    float* c = static_cast<float*>(p.c);
    if (p.b_layout == NANOVLLM_GEMM_B_NK)
        hipLaunchKernelGGL(fp32_tiled_kernel<NANOVLLM_GEMM_B_NK>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                           p.lda, p.ldb, p.ldc, int(tiles_m), int(tiles_n));
    else
        hipLaunchKernelGGL(fp32_tiled_kernel<NANOVLLM_GEMM_B_KN>, grid, block, 0, s, a, b, c, p.m, p.n, p.k,
                           p.lda, p.ldb, p.ldc, int(tiles_m), int(tiles_n));
    return check_launch("fp32_tiled");
}

}  // namespace nvg
