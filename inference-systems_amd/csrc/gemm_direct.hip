// mfma_direct: BF16/FP16 GEMM with one wave per 32x32 output tile and the
// matrix-core operands read straight from global memory (no LDS).  It is
// the MI355X rung that corresponds to the reference's direct WMMA kernels
// (cuda_kernels/gemm/src/gemm_bench.cu:80-115 with B[K,N];
// gemm_wmma.cu:56-104 with B = W[N,K]) and also covers what they skip:
// partial tiles (gemm_bench.cu:92), K that is not a multiple of 16, odd
// strides and unaligned pointers.  It is the selection table's fallback for
// any half-precision problem the faster kernels cannot take.
#include "gemm_common.hpp"

namespace nvg {
namespace {

// 8 consecutive 16-bit elements p[0..7] of which only the first `valid`
// are read; the rest are zero.  Packed as a 16-byte MFMA operand.
__device__ __forceinline__ u32x4_t load8_masked(const uint16_t* p, int64_t valid) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = (2 * i < valid) ? p[2 * i] : 0u;
        const uint32_t hi = (2 * i + 1 < valid) ? p[2 * i + 1] : 0u;
        w[i] = lo | (hi << 16);
    }
    return u32x4_t{w[0], w[1], w[2], w[3]};
}

// 8 elements p[0], p[stride], ..., p[7*stride], the first `valid` read.
__device__ __forceinline__ u32x4_t load8_strided(const uint16_t* p, int64_t stride, int64_t valid) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = (2 * i < valid) ? p[(2 * i) * stride] : 0u;
        const uint32_t hi = (2 * i + 1 < valid) ? p[(2 * i + 1) * stride] : 0u;
        w[i] = lo | (hi << 16);
    }
    return u32x4_t{w[0], w[1], w[2], w[3]};
}

// FAST: A rows (and W[N,K] rows) can be read as aligned 16-byte chunks.
// Then the K loop runs in groups of kUnroll steps whose loads are all issued
// (from row addresses clamped into the matrix) before the group's MFMAs, so
// each lane keeps kUnroll steps of operands in flight instead of waiting
// out one load latency per 16-element step; rows outside the matrix are
// zeroed after the loads.  A K tail shorter than a group takes the general
// loop.
constexpr int kUnroll = 4;

template <int DT, int DT_OUT, int BL, int FAST>
__global__ __launch_bounds__(256) void mfma_direct_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n, int vec_a, int vec_b) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int half = lane >> 5;
    const int r32 = lane & 31;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int64_t m0 = int64_t(tm) * 64 + (wave >> 1) * 32;
    const int64_t n0 = int64_t(tn) * 64 + (wave & 1) * 32;

    // Lane l feeds A row (m0 + l%32) and B column (n0 + l%32), K-chunk l/32.
    const int64_t arow = m0 + r32;
    const int64_t bcol = n0 + r32;
    const bool a_in = arow < m;
    const bool b_in = bcol < n;
    const uint16_t* ap = a + (a_in ? arow : 0) * lda;

    f32x16_t acc = {};
    int64_t k0 = 0;
    if constexpr (FAST) {
        const u32x4_t zero = {0u, 0u, 0u, 0u};
        const uint16_t* bp = BL == NANOVLLM_GEMM_B_NK ? b + (b_in ? bcol : 0) * ldb : b + (b_in ? bcol : 0);
        for (; k0 + 16 * kUnroll <= k; k0 += 16 * kUnroll) {
            u32x4_t af[kUnroll], bf[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t kb = k0 + 16 * u + 8 * half;
                af[u] = load16(ap + kb);
                if constexpr (BL == NANOVLLM_GEMM_B_NK) bf[u] = load16(bp + kb);
                else bf[u] = load8_strided(bp + kb * ldb, ldb, 8);
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                acc = mfma_32x32x16<DT>(a_in ? af[u] : zero, b_in ? bf[u] : zero, acc);
        }
    }
    for (; k0 < k; k0 += 16) {
        const int64_t kb = k0 + 8 * half;
        const int64_t kvalid = k - kb;  // may be <= 0 for the tail chunk
        u32x4_t af, bf;
        if (!a_in || kvalid <= 0) {
            af = u32x4_t{0u, 0u, 0u, 0u};
        } else if (vec_a && kvalid >= 8) {
            af = load16(ap + kb);
        } else {
            af = load8_masked(ap + kb, kvalid);
        }
        if (!b_in || kvalid <= 0) {
            bf = u32x4_t{0u, 0u, 0u, 0u};
        } else if constexpr (BL == NANOVLLM_GEMM_B_NK) {
            const uint16_t* bp = b + bcol * ldb + kb;
            bf = (vec_b && kvalid >= 8) ? load16(bp) : load8_masked(bp, kvalid);
        } else {
            bf = load8_strided(b + kb * ldb + bcol, ldb, kvalid);
        }
        acc = mfma_32x32x16<DT>(af, bf, acc);
    }

#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + 8 * (v >> 2) + 4 * half + (v & 3);
        if (row < m && b_in) store_elem<DT_OUT>(c, row * ldc + bcol, acc[v]);
    }
}

template <int DT, int DT_OUT>
int launch_typed(const Problem& p, hipStream_t s) {
    const int64_t tiles_m = (p.m + 63) / 64, tiles_n = (p.n + 63) / 64;
    if (tiles_m * tiles_n > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "mfma_direct: grid too large");
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n)), block(256);
    const auto* a = static_cast<const uint16_t*>(p.a);
    const auto* b = static_cast<const uint16_t*>(p.b);
    const int vec_a = (reinterpret_cast<uintptr_t>(p.a) % 16 == 0) && (p.lda % 8 == 0);
    const int vec_b = (reinterpret_cast<uintptr_t>(p.b) % 16 == 0) && (p.ldb % 8 == 0);
    const int ti = int(tiles_m), tj = int(tiles_n);
    if (p.b_layout == NANOVLLM_GEMM_B_NK) {
        if (vec_a && vec_b)
            hipLaunchKernelGGL((mfma_direct_kernel<DT, DT_OUT, NANOVLLM_GEMM_B_NK, 1>), grid, block, 0, s, a, b, p.c,
                               p.m, p.n, p.k, p.lda, p.ldb, p.ldc, ti, tj, vec_a, vec_b);
        else
            hipLaunchKernelGGL((mfma_direct_kernel<DT, DT_OUT, NANOVLLM_GEMM_B_NK, 0>), grid, block, 0, s, a, b, p.c,
                               p.m, p.n, p.k, p.lda, p.ldb, p.ldc, ti, tj, vec_a, vec_b);
    } else {
        if (vec_a)
            hipLaunchKernelGGL((mfma_direct_kernel<DT, DT_OUT, NANOVLLM_GEMM_B_KN, 1>), grid, block, 0, s, a, b, p.c,
                               p.m, p.n, p.k, p.lda, p.ldb, p.ldc, ti, tj, vec_a, vec_b);
        else
            hipLaunchKernelGGL((mfma_direct_kernel<DT, DT_OUT, NANOVLLM_GEMM_B_KN, 0>), grid, block, 0, s, a, b, p.c,
                               p.m, p.n, p.k, p.lda, p.ldb, p.ldc, ti, tj, vec_a, vec_b);
    }
    return check_launch("mfma_direct");
}

}  // namespace

int launch_mfma_direct(const Problem& p, hipStream_t s) {
    if (p.dtype_in == NANOVLLM_GEMM_BF16) {
        if (p.dtype_out == NANOVLLM_GEMM_BF16) return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_BF16>(p, s);
        return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_F32>(p, s);
    }
    if (p.dtype_out == NANOVLLM_GEMM_F16) return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F16>(p, s);
    return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F32>(p, s);
}

}  // namespace nvg
