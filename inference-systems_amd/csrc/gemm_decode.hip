// splitk_decode: the bandwidth-bound small-M GEMM (M <= 32), C = A * W^T
// with W[N,K] in the nn.Linear layout.  At these shapes the work is
// streaming W once from HBM (N*K*2 bytes) while A (M*K*2 bytes, at most
// 64 KiB) stays in L2.  Design:
//   * one 256-thread workgroup per 16 rows of W; its 4 waves split K,
//     taking 32-element K-steps round robin (wave w takes steps w, w+4, ..),
//     so together the 4 waves read 256 contiguous bytes of each W row;
//   * each lane issues all of its W loads (8 x 16 B for K = 1024) before
//     the first MFMA, so the whole of W is in flight almost at once;
//   * v_mfma_f32_16x16x32 with W as the first operand (16 rows of W) and up
//     to two 16-row groups of A as the second; rows of A past M are zero;
//   * the four per-wave partial tiles are summed in LDS in a fixed order
//     (deterministic, no atomics, no workspace) and written once.
// It replaces the reference's cuBLAS fallback for decode shapes and the
// M == 16 direct-WMMA special case (cuda_kernels/gemm/src/gemm_bench.cu:260-273).
#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kDecWaves = 4;
constexpr int kDecRows = 16;   // W rows per workgroup
constexpr int kDecStep = 32;   // K elements per MFMA
constexpr int kDecUnroll = 8;  // K-steps whose loads are issued together

template <int DT, int DT_OUT, int MG>
__global__ __launch_bounds__(256) void splitk_decode_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc) {
    __shared__ float red[kDecWaves][MG][kDecRows][16];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i16 = lane & 15;   // W row (first operand) / A row (second operand)
    const int grp = lane >> 4;   // which 8-element chunk of the 32-wide K-step

    const int64_t n0 = int64_t(blockIdx.x) * kDecRows;
    const int64_t wrow = min(n0 + i16, n - 1);
    const uint16_t* wp = w + wrow * ldb + grp * 8;
    const uint16_t* ap[MG];
    bool a_in[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) {
        const int64_t arow = g * 16 + i16;
        a_in[g] = arow < m;
        ap[g] = a + (a_in[g] ? arow : 0) * lda + grp * 8;
    }

    const int64_t steps = (k + kDecStep - 1) / kDecStep;
    f32x4_t acc[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) acc[g] = f32x4_t{};

    for (int64_t s0 = wave; s0 < steps; s0 += kDecWaves * kDecUnroll) {
        u32x4_t wf[kDecUnroll];
        u32x4_t af[MG][kDecUnroll];
#pragma unroll
        for (int u = 0; u < kDecUnroll; ++u) {
            const int64_t kc = (s0 + kDecWaves * u) * kDecStep + grp * 8;
            const bool in_k = kc < k;  // K % 8 == 0: a chunk is all in or all out
            wf[u] = in_k ? load16(wp + (kc - grp * 8)) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
            for (int g = 0; g < MG; ++g)
                af[g][u] = (in_k && a_in[g]) ? load16(ap[g] + (kc - grp * 8)) : u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kDecUnroll; ++u)
#pragma unroll
            for (int g = 0; g < MG; ++g) acc[g] = mfma_16x16x32<DT>(wf[u], af[g][u], acc[g]);
    }

    // acc[g][v] is D[n = 4*(l/16) + v][m = l%16] of group g.
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[wave][g][4 * grp + v][i16] = acc[g][v];
    __syncthreads();

    const int t = threadIdx.x;
    const int nn = t & 15;
    const int mm = t >> 4;
#pragma unroll
    for (int g = 0; g < MG; ++g) {
        const float sum = ((red[0][g][nn][mm] + red[1][g][nn][mm]) + red[2][g][nn][mm]) + red[3][g][nn][mm];
        const int64_t row = g * 16 + mm;
        const int64_t col = n0 + nn;
        if (row < m && col < n) store_elem<DT_OUT>(c, row * ldc + col, sum);
    }
}

template <int DT, int DT_OUT>
int launch_typed(const Problem& p, hipStream_t s) {
    const int64_t blocks = (p.n + kDecRows - 1) / kDecRows;
    if (blocks > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "splitk_decode: grid too large");
    const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
    const auto* a = static_cast<const uint16_t*>(p.a);
    const auto* w = static_cast<const uint16_t*>(p.b);
    if (p.m <= 16)
        hipLaunchKernelGGL((splitk_decode_kernel<DT, DT_OUT, 1>), grid, block, 0, s, a, w, p.c, p.m, p.n, p.k,
                           p.lda, p.ldb, p.ldc);
    else
        hipLaunchKernelGGL((splitk_decode_kernel<DT, DT_OUT, 2>), grid, block, 0, s, a, w, p.c, p.m, p.n, p.k,
                           p.lda, p.ldb, p.ldc);
    return check_launch("splitk_decode");
}

}  // namespace

int launch_splitk_decode(const Problem& p, hipStream_t s) {
    if (p.dtype_in == NANOVLLM_GEMM_BF16) {
        if (p.dtype_out == NANOVLLM_GEMM_BF16) return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_BF16>(p, s);
        return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_F32>(p, s);
    }
    if (p.dtype_out == NANOVLLM_GEMM_F16) return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F16>(p, s);
    return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F32>(p, s);
}

}  // namespace nvg
