// gemv_decode: the M = 1 GEMM (single-token decode), c[n] = sum_k a[k] W[n,k]
// with W[N,K] in the nn.Linear layout.  Pure streaming of W: one wave per W
// row, each lane reading 16-byte chunks of that row (a wave instruction covers
// 1 KiB of one row, fully coalesced), fp32 multiply-adds on the VALU, then a
// fixed-order DPP sum across the 64 lanes.  Many small workgroups (4 rows
// each) keep W requests spread over every HBM channel from the first cycle;
// measured on MI355X this streams 12.6 MB noticeably faster than the MFMA
// decode kernel, whose 16-row tiles waste 15/16 of each MFMA at M = 1.
// Replaces the reference's cuBLAS path for the decode shape
// (cuda_kernels/gemm/src/gemm_bench.cu:45, qwen35_decode_qkv, dispatch
// "cublas" in results/rtx3060_gemm_matrix.csv:2-3).
#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kGemvRows = 4;     // W rows per 256-thread workgroup (one per wave)

template <int DT>
__device__ __forceinline__ float dot8(u32x4_t av, u32x4_t wv, float s) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        s = __builtin_fmaf(half_to_f32<DT>(uint16_t(av[q])), half_to_f32<DT>(uint16_t(wv[q])), s);
        s = __builtin_fmaf(half_to_f32<DT>(uint16_t(av[q] >> 16)), half_to_f32<DT>(uint16_t(wv[q] >> 16)), s);
    }
    return s;
}

// Sum over the 64 lanes of a wave, the same value in every lane, in a fixed
// order: inside each 16-lane row by DPP moves (pairs of lanes i ^ 1, i ^ 2,
// then the mirrored half row and row; each pair adds a + b and b + a, which
// are equal, so all 16 lanes hold the same row sum), then the four row sums
// read as scalars and added as (r0 + r1) + (r2 + r3).  DPP moves run on the
// VALU; the lane shuffles they replace went through the LDS crossbar with a
// wait per step (M = 1, 6144 x 1024: 3.96 -> 3.77 us without any reduction).
__device__ __forceinline__ float wave_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    const int bits = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 48));
    return (r0 + r1) + (r2 + r3);
}

// U: 16-byte chunks per lane whose loads are issued together, chosen so a
// K of 64 U chunks is one trip without loads predicated off (the sum order,
// chunk lane, lane + 64, ..., does not depend on U).
template <int DT, int DT_OUT, int EPI, int U>
__global__ __launch_bounds__(256) void gemv_decode_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t n, int64_t k, int64_t ldb) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kGemvRows + (threadIdx.x >> 6);   // output column
    const uint16_t* wr = w + min_i64(row, n - 1) * ldb;
    // EPI_SILU_MUL: the wave also streams the up row of its column (row n + j
    // of W = [W_gate; W_up]).
    const uint16_t* wu = EPI == EPI_SILU_MUL ? w + (n + min_i64(row, n - 1)) * ldb : wr;
    const int64_t chunks = k / 8;   // K % 8 == 0 is required by the selection table

    float acc = 0.0f, acc_up = 0.0f;
    for (int64_t c0 = lane; c0 < chunks; c0 += 64 * U) {
        u32x4_t wv[U], uv[U], av[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t cc = c0 + 64 * u;
            const bool in = cc < chunks;
            wv[u] = in ? load16(wr + cc * 8) : u32x4_t{0u, 0u, 0u, 0u};
            if constexpr (EPI == EPI_SILU_MUL) uv[u] = in ? load16(wu + cc * 8) : u32x4_t{0u, 0u, 0u, 0u};
            av[u] = in ? load16(a + cc * 8) : u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc = dot8<DT>(av[u], wv[u], acc);
            if constexpr (EPI == EPI_SILU_MUL) acc_up = dot8<DT>(av[u], uv[u], acc_up);
        }
    }
    acc = wave_sum(acc);
    if constexpr (EPI == EPI_SILU_MUL) acc_up = wave_sum(acc_up);
    if (lane == 0 && row < n) {
        if constexpr (EPI == EPI_SILU_MUL) store_elem<DT_OUT>(c, row, silu_f32(acc) * acc_up);
        else store_elem<DT_OUT>(c, row, acc);
    }
}

template <int DT, int DT_OUT, int U>
void launch_unrolled(const Problem& p, dim3 grid, hipStream_t s) {
    const auto* ap = static_cast<const uint16_t*>(p.a);
    const auto* wp = static_cast<const uint16_t*>(p.b);
    if (p.epi == EPI_SILU_MUL)
        hipLaunchKernelGGL((gemv_decode_kernel<DT, DT_OUT, EPI_SILU_MUL, U>), grid, dim3(256), 0, s, ap, wp, p.c, p.n,
                           p.k, p.ldb);
    else
        hipLaunchKernelGGL((gemv_decode_kernel<DT, DT_OUT, EPI_NONE, U>), grid, dim3(256), 0, s, ap, wp, p.c, p.n,
                           p.k, p.ldb);
}

// Loads issued together per lane: as many as its chunks of one row, up to 4
// (measured on MI355X, N x K = 6144 x 1024: 4.21 us with 2 against 4.43 us
// with 4, two of them predicated off; 1024 x 3584: 3.99 us with 4 against
// 4.72 us with 2).
template <int DT, int DT_OUT>
int launch_typed(const Problem& p, hipStream_t s) {
    const int64_t blocks = (p.n + kGemvRows - 1) / kGemvRows;
    if (blocks > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "gemv_decode: grid too large");
    const dim3 grid(static_cast<uint32_t>(blocks));
    const int64_t per_lane = (p.k / 8 + 63) / 64;
    if (per_lane <= 1) launch_unrolled<DT, DT_OUT, 1>(p, grid, s);
    else if (per_lane == 2) launch_unrolled<DT, DT_OUT, 2>(p, grid, s);
    else launch_unrolled<DT, DT_OUT, 4>(p, grid, s);
    return check_launch("gemv_decode");
}

}  // namespace

int launch_gemv_decode(const Problem& p, hipStream_t s) {
    if (p.dtype_in == NANOVLLM_GEMM_BF16) {
        if (p.dtype_out == NANOVLLM_GEMM_BF16) return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_BF16>(p, s);
        return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_F32>(p, s);
    }
    if (p.dtype_out == NANOVLLM_GEMM_F16) return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F16>(p, s);
    return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F32>(p, s);
}

}  // namespace nvg
