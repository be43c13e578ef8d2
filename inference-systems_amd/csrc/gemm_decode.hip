// splitk_decode: the bandwidth-bound small-M GEMM (M <= 32), C = A * W^T
// with W[N,K] in the nn.Linear layout.  At these shapes the work is
// streaming W once from HBM (N*K*2 bytes) while A (M*K*2 bytes, at most
// 64 KiB) stays in L2.  Design:
//   * one workgroup per 16 rows of W (4 waves; M <= 8), per 32 rows (8
//     waves; 8 < M <= 32, so each A fragment serves two W row groups) or,
//     for very wide W, per 64 rows (4 waves); the waves split K, taking
//     32-element K-steps round robin, so together they read contiguous runs
//     of each W row;
//   * each lane issues its W loads for several K-steps (8 x 16 B for K = 1024
//     with 4 waves) before the first MFMA, so W is in flight almost at once;
//   * v_mfma_f32_16x16x32 with W as the first operand (16 rows of W) and up
//     to two 16-row groups of A as the second; rows of A past M are zero;
//   * the four per-wave partial tiles are summed in LDS in a fixed order
//     (deterministic, no atomics, no workspace) and written once.
// It replaces the reference's cuBLAS fallback for decode shapes and the
// M == 16 direct-WMMA special case (cuda_kernels/gemm/src/gemm_bench.cu:260-273).
#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kDecStep = 32;   // K elements per MFMA

// RG groups of 16 W rows per workgroup, WAVES waves splitting K round robin,
// MG groups of 16 A rows, UNROLL K-steps whose loads are issued together.
template <int DT, int DT_OUT, int MG, int RG, int WAVES, int UNROLL, int EPI>
__global__ __launch_bounds__(WAVES * 64) void splitk_decode_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, uint64_t* __restrict__ keys) {
    __shared__ float red[WAVES][RG][MG][16][16];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i16 = lane & 15;   // W row (first operand) / A row (second operand)
    const int grp = lane >> 4;   // which 8-element chunk of the 32-wide K-step

    // EPI_SILU_MUL: W-row groups pair up, group 2s holding gate rows and
    // group 2s + 1 the up rows of the same 16 output columns.
    static_assert(EPI != EPI_SILU_MUL || RG % 2 == 0, "gate/up group pairs");
    constexpr int OG = EPI == EPI_SILU_MUL ? RG / 2 : RG;   // 16-column output groups per workgroup
    const int64_t n0 = int64_t(blockIdx.x) * 16 * OG;         // first output column
    const uint16_t* wp[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
        if constexpr (EPI == EPI_SILU_MUL)
            wp[r] = w + ((r & 1) ? n : 0) * ldb + min_i64(n0 + 16 * (r >> 1) + i16, n - 1) * ldb + grp * 8;
        else
            wp[r] = w + min_i64(n0 + 16 * r + i16, n - 1) * ldb + grp * 8;
    }
    const uint16_t* ap[MG];
    bool a_in[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) {
        const int64_t arow = g * 16 + i16;
        a_in[g] = arow < m;
        ap[g] = a + (a_in[g] ? arow : 0) * lda + grp * 8;
    }

    const int64_t steps = (k + kDecStep - 1) / kDecStep;
    f32x4_t acc[RG][MG];
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[r][g] = f32x4_t{};

    for (int64_t s0 = wave; s0 < steps; s0 += WAVES * UNROLL) {
        u32x4_t wf[RG][UNROLL];
        u32x4_t af[MG][UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t ks = (s0 + WAVES * u) * kDecStep;
            const bool in_k = ks + grp * 8 < k;  // K % 8 == 0: a chunk is all in or all out
#pragma unroll
            for (int r = 0; r < RG; ++r) wf[r][u] = in_k ? load16(wp[r] + ks) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
            for (int g = 0; g < MG; ++g)
                af[g][u] = (in_k && a_in[g]) ? load16(ap[g] + ks) : u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
#pragma unroll
            for (int r = 0; r < RG; ++r)
#pragma unroll
                for (int g = 0; g < MG; ++g) acc[r][g] = mfma_16x16x32<DT>(wf[r][u], af[g][u], acc[r][g]);
    }

    // acc[r][g][v] is D[n = 4*(l/16) + v][m = l%16] of W-row group r, A-row group g.
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int g = 0; g < MG; ++g)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[wave][r][g][4 * grp + v][i16] = acc[r][g][v];
    __syncthreads();

    if constexpr (EPI == EPI_ARGMAX) {
        // Per row of A, the best of this workgroup's 16 * RG columns: the
        // sums go to LDS, then one thread per row scans them.
        __shared__ float vals[MG * 16][16 * RG + 1];
        for (int e = threadIdx.x; e < RG * MG * 256; e += WAVES * 64) {
            const int r = e / (MG * 256);
            const int g = (e / 256) % MG;
            const int nn = e & 15;
            const int mm = (e >> 4) & 15;
            float sum = red[0][r][g][nn][mm];
#pragma unroll
            for (int wv = 1; wv < WAVES; ++wv) sum += red[wv][r][g][nn][mm];
            vals[g * 16 + mm][16 * r + nn] = sum;
        }
        __syncthreads();
        const int row = threadIdx.x;
        if (row < MG * 16 && row < m) {
            uint64_t best = 0;
            for (int cc = 0; cc < 16 * RG; ++cc) {
                if (n0 + cc >= n) break;
                const uint64_t key = argmax_key(vals[row][cc], n0 + cc);
                best = key > best ? key : best;
            }
            keys[row * int64_t(gridDim.x) + blockIdx.x] = best;
        }
        return;
    }

    // Sum the per-wave partials in wave order (deterministic) and store.
    for (int e = threadIdx.x; e < OG * MG * 256; e += WAVES * 64) {
        const int o = e / (MG * 256);
        const int g = (e / 256) % MG;
        const int nn = e & 15;
        const int mm = (e >> 4) & 15;
        const int64_t row = g * 16 + mm;
        const int64_t col = n0 + 16 * o + nn;
        if constexpr (EPI == EPI_SILU_MUL) {
            float gate = red[0][2 * o][g][nn][mm], up = red[0][2 * o + 1][g][nn][mm];
#pragma unroll
            for (int wv = 1; wv < WAVES; ++wv) {
                gate += red[wv][2 * o][g][nn][mm];
                up += red[wv][2 * o + 1][g][nn][mm];
            }
            if (row < m && col < n) store_elem<DT_OUT>(c, row * ldc + col, silu_f32(gate) * up);
        } else {
            float sum = red[0][o][g][nn][mm];
#pragma unroll
            for (int wv = 1; wv < WAVES; ++wv) sum += red[wv][o][g][nn][mm];
            if (row < m && col < n) store_elem<DT_OUT>(c, row * ldc + col, sum);
        }
    }
}

template <int DT, int DT_OUT, int MG, int RG, int WAVES, int UNROLL, int EPI = EPI_NONE>
int launch_cfg(const Problem& p, hipStream_t s) {
    constexpr int OG = EPI == EPI_SILU_MUL ? RG / 2 : RG;
    const int64_t blocks = (p.n + 16 * OG - 1) / (16 * OG);
    if (blocks > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "splitk_decode: grid too large");
    const dim3 grid(static_cast<uint32_t>(blocks)), block(WAVES * 64);
    if (EPI == EPI_ARGMAX) *p.key_blocks = blocks;
    hipLaunchKernelGGL((splitk_decode_kernel<DT, DT_OUT, MG, RG, WAVES, UNROLL, EPI>), grid, block, 0, s,
                       static_cast<const uint16_t*>(p.a), static_cast<const uint16_t*>(p.b), p.c, p.m, p.n, p.k,
                       p.lda, p.ldb, p.ldc, p.keys);
    return check_launch("splitk_decode");
}

// Configurations measured on MI355X, K = 1024.
//   N = 6144: up to 8 rows of A, 16 W rows per 4-wave workgroup; beyond that
//   32 W rows per 8-wave workgroup, which reads each A fragment once for two
//   W row groups (M = 16: 5.9 us, M = 32: 7.2 us).
//   N >= 65536 (LM head, 151936 rows): every workgroup reads all of A from
//   L2, so for M > 1 a workgroup takes 64 W rows with 4 waves, which cuts
//   that traffic 4x against 16 rows (M = 8 / 16 / 32: 61 / 66 / 76 us,
//   against 64 / 70 / 81 us); M = 1 keeps the 16-row workgroups (51 us).
constexpr int64_t kWideN = 65536;

// Fused gate/up + SiLU-and-mul: W-row groups come in gate/up pairs, so the
// workgroups take 2 (or, for very wide W, 4) groups of 16 rows.
template <int DT, int DT_OUT>
int launch_silu_mul(const Problem& p, hipStream_t s) {
    const bool wide = 2 * p.n >= kWideN;
    if (p.m <= 16) {
        if (wide) return launch_cfg<DT, DT_OUT, 1, 4, 4, 4, EPI_SILU_MUL>(p, s);
        return launch_cfg<DT, DT_OUT, 1, 2, 4, 4, EPI_SILU_MUL>(p, s);
    }
    if (wide) return launch_cfg<DT, DT_OUT, 2, 4, 4, 4, EPI_SILU_MUL>(p, s);
    return launch_cfg<DT, DT_OUT, 2, 2, 8, 2, EPI_SILU_MUL>(p, s);
}

// Greedy LM head: the plain configurations, writing partial keys instead of
// the fp32 logits.
template <int DT>
int launch_argmax(const Problem& p, hipStream_t s) {
    constexpr int F = NANOVLLM_GEMM_F32;
    const bool wide = p.n >= kWideN && p.m > 1;
    if (p.m <= 8) {
        if (wide) return launch_cfg<DT, F, 1, 4, 4, 4, EPI_ARGMAX>(p, s);
        return launch_cfg<DT, F, 1, 1, 4, 8, EPI_ARGMAX>(p, s);
    }
    if (p.m <= 16) {
        if (wide) return launch_cfg<DT, F, 1, 4, 4, 4, EPI_ARGMAX>(p, s);
        return launch_cfg<DT, F, 1, 2, 8, 2, EPI_ARGMAX>(p, s);
    }
    if (wide) return launch_cfg<DT, F, 2, 4, 4, 4, EPI_ARGMAX>(p, s);
    return launch_cfg<DT, F, 2, 2, 8, 2, EPI_ARGMAX>(p, s);
}

template <int DT, int DT_OUT>
int launch_typed(const Problem& p, hipStream_t s) {
    if (p.epi == EPI_SILU_MUL) return launch_silu_mul<DT, DT_OUT>(p, s);
    const bool wide = p.n >= kWideN && p.m > 1;
    if (p.m <= 8) {
        if (wide) return launch_cfg<DT, DT_OUT, 1, 4, 4, 4>(p, s);
        return launch_cfg<DT, DT_OUT, 1, 1, 4, 8>(p, s);
    }
    if (p.m <= 16) {
        if (wide) return launch_cfg<DT, DT_OUT, 1, 4, 4, 4>(p, s);
        return launch_cfg<DT, DT_OUT, 1, 2, 8, 2>(p, s);
    }
    if (wide) return launch_cfg<DT, DT_OUT, 2, 4, 4, 4>(p, s);
    return launch_cfg<DT, DT_OUT, 2, 2, 8, 2>(p, s);
}

}  // namespace

int launch_splitk_decode(const Problem& p, hipStream_t s) {
    if (p.epi == EPI_ARGMAX) {
        if (p.dtype_in == NANOVLLM_GEMM_BF16) return launch_argmax<NANOVLLM_GEMM_BF16>(p, s);
        return launch_argmax<NANOVLLM_GEMM_F16>(p, s);
    }
    if (p.dtype_in == NANOVLLM_GEMM_BF16) {
        if (p.dtype_out == NANOVLLM_GEMM_BF16) return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_BF16>(p, s);
        return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_F32>(p, s);
    }
    if (p.dtype_out == NANOVLLM_GEMM_F16) return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F16>(p, s);
    return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F32>(p, s);
}

}  // namespace nvg
