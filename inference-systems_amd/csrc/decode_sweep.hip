// Configuration sweep of the decode kernels behind `bench.py --decode-sweep`:
// every configuration listed below of the LDS-staged splitk_decode kernel
// and of the register-loading splitk_lines kernel (defined here), each
// launchable on its own (bf16 in and out, plain store, W[N,K], dense leading
// dimensions), so the configuration table in gemm_decode.hip can be
// re-measured on the device.  A library of its own (libnanovllm_decode_sweep.so), built from the
// same kernel templates as the GEMM library.
//   lds   rows = rows of A per copy, rg = W rows per workgroup, waves, lpb =
//         lines per wave copied together (16 K partitions; with `parts=P`,
//         P partitions, the counts of the LM-head configurations)
//   areg  splitk_decode with A's fragments loaded from global memory straight
//         into registers (only W copied into LDS): rows of A, rg, waves, lpb
//   kn    the B[K,N] form of splitk_decode: rows of A per copy, 64 columns
//         per workgroup, waves, lpb (16 partitions with 16 waves, 8 with 8)
//   lines rows = rows of A loaded per line, rg = W rows per workgroup, waves,
//         lpb = lines per wave loaded together (16 K partitions); the
//         register-loading kernel below, which the GEMM library does not use
#include <cstdarg>
#include <cstdio>

#include "decode_kernels.hpp"

namespace nvg {

int set_error(int code, const char*, ...) { return code; }

int check_launch(const char*) {
    return hipGetLastError() == hipSuccess ? NANOVLLM_GEMM_OK : NANOVLLM_GEMM_ELAUNCH;
}

namespace {

constexpr int BF = NANOVLLM_GEMM_BF16;

// splitk_lines: a register-loading alternative to splitk_decode, measured
// here and not used by the GEMM library.
//   * Lane l = 16 g + 8 h + r of a load takes chunk 4 h + g (16 bytes) of
//     line L of row r of an 8-row group, so one instruction reads 8 whole
//     lines (1 KiB) straight into registers, nothing passing through LDS.
//   * Used as the first operand of v_mfma_f32_16x16x32 that register is row
//     i = 8 h + r with k-group g; A's 8-row groups are loaded the same way
//     and used as the second operand (column j = 8 h' + m').  The product's
//     diagonal blocks h = h' are the two half lines of W row r times A row
//     m', D[r][m'] for chunks 0-3 and D[8 + r][8 + m'] for chunks 4-7; the
//     off-diagonal blocks are discarded (one MFMA per KiB of W at M <= 8,
//     four at M = 32).
//   * Waves split K by lines (line L accumulates into partition L % 16,
//     16 / WAVES partitions per wave, LPB lines' loads issued together);
//     the partition tiles meet in LDS and are added in partition order.
// On MI355X (N = 6144, K = 1024, W streamed from HBM) every configuration
// ran slower than splitk_decode's LDS-staged copies: 4.6-5.3 against
// 4.4-4.5 us at M <= 8, 6.4 against 4.7 us at M = 16 and 8.4 against
// 5.5 us at M = 32; adding the half lines with a lane shuffle before the
// LDS reduction instead of in it was slower still.  AG: 8-row groups of A;
// RG: 8-row groups of W per workgroup.  K % 8 == 0; chunks past K load zeros.
constexpr int kLineParts = 16;

template <int DT, int DT_OUT, int AG, int RG, int WAVES, int LPB>
__global__ __launch_bounds__(WAVES * 64) void splitk_lines_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc) {
    static_assert(AG == 1 || AG == 2 || AG == 4, "8, 16 or 32 rows of A");
    static_assert(kLineParts % WAVES == 0, "whole partitions per wave");
    constexpr int PW = kLineParts / WAVES;             // partitions per wave
    constexpr int ROUND = LPB > PW ? LPB : PW;         // lines per wave per loop trip
    static_assert(ROUND % LPB == 0 && ROUND % PW == 0, "load batches and partitions tile a trip");
    constexpr int TILE = 128;   // kept floats of one product: 2 half lines x 8 W rows x 8 A rows
    __shared__ float part[WAVES][PW * RG * AG * TILE];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r8 = lane & 7;
    const int cofs = 8 * (4 * ((lane >> 3) & 1) + (lane >> 4));   // element offset of the lane's chunk
    const int64_t n0 = int64_t(blockIdx.x) * 8 * RG;              // first output column
    const uint16_t* wsrc[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) wsrc[r] = w + min_i64(n0 + 8 * r + r8, n - 1) * ldb + cofs;
    const uint16_t* asrc[AG];
#pragma unroll
    for (int g = 0; g < AG; ++g) asrc[g] = a + min_i64(8 * g + r8, m - 1) * lda + cofs;

    const int64_t lines = (k + kLine - 1) / kLine;
    f32x4_t acc[PW][RG][AG];
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int r = 0; r < RG; ++r)
#pragma unroll
            for (int g = 0; g < AG; ++g) acc[q][r][g] = f32x4_t{};

    // Wave w takes lines w + WAVES j, j = 0, 1, ...; line j of a trip goes to
    // partition w + WAVES (j % PW) (= line % 16, as WAVES * ROUND is a
    // multiple of 16), in batches of LPB lines loaded together.
    for (int64_t l0 = wave; l0 < lines; l0 += int64_t(WAVES) * ROUND) {
#pragma unroll
        for (int bt = 0; bt < ROUND / LPB; ++bt) {
            if (l0 + int64_t(WAVES) * (bt * LPB) >= lines) break;
            u32x4_t wf[LPB][RG], af[LPB][AG];
#pragma unroll
            for (int t = 0; t < LPB; ++t) {
                const int64_t line = l0 + int64_t(WAVES) * (bt * LPB + t);
                const bool in = line < lines && line * kLine + cofs < k;
#pragma unroll
                for (int r = 0; r < RG; ++r)
                    wf[t][r] = in ? load16(wsrc[r] + line * kLine) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
                for (int g = 0; g < AG; ++g)
                    af[t][g] = in ? load16(asrc[g] + line * kLine) : u32x4_t{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int t = 0; t < LPB; ++t) {
                const int64_t line = l0 + int64_t(WAVES) * (bt * LPB + t);
                if (line >= lines) break;
                const int q = (bt * LPB + t) % PW;   // compile-time after unrolling
#pragma unroll
                for (int r = 0; r < RG; ++r)
#pragma unroll
                    for (int g = 0; g < AG; ++g) acc[q][r][g] = mfma_16x16x32<DT>(wf[t][r], af[t][g], acc[q][r][g]);
            }
        }
    }

    // acc[q][r][g][v] of lane l is D[i = 4 (l / 16) + v][j = l % 16]: kept
    // when i and j lie in the same half (h = l / 32 = j / 8), as element
    // (h, A row j % 8, W row i % 8) of the wave's tile for (q, r, g).
    {
        const int hh = lane >> 5, j = lane & 15;
        if ((j >> 3) == hh) {
            const int mm = j & 7, ri = 4 * ((lane >> 4) & 1);
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int r = 0; r < RG; ++r)
#pragma unroll
                    for (int g = 0; g < AG; ++g)
#pragma unroll
                        for (int v = 0; v < 4; ++v)
                            part[wave][((q * RG + r) * AG + g) * TILE + (hh * 8 + mm) * 8 + ri + v] = acc[q][r][g][v];
        }
    }
    __syncthreads();
    // Output (A row ar, column n0 + cw): partition p sits in wave p % WAVES, slot p / WAVES.
    auto total = [&](int cw, int ar) {
        const int r = cw >> 3, ri = cw & 7, g = ar >> 3, mm = ar & 7;
        auto half_sum = [&](int p) {
            const float* t = &part[p % WAVES][(((p / WAVES) * RG + r) * AG + g) * TILE + mm * 8 + ri];
            return t[0] + t[64];
        };
        float sum = half_sum(0);
#pragma unroll
        for (int p = 1; p < kLineParts; ++p) sum += half_sum(p);
        return sum;
    };

    for (int e = threadIdx.x; e < RG * AG * 64; e += WAVES * 64) {
        const int cw = e % (8 * RG), ar = e / (8 * RG);
        const int64_t col = n0 + cw;
        if (ar >= m || col >= n) continue;
        store_elem<DT_OUT>(c, ar * ldc + col, total(cw, ar));
    }
}

template <int AG, int RG, int WAVES, int LPB>
int launch_lines(const Problem& p, hipStream_t s) {
    if (p.m > 8 * AG) return NANOVLLM_GEMM_EUNSUPPORTED;
    const int64_t blocks = (p.n + 8 * RG - 1) / (8 * RG);
    if (blocks > INT32_MAX) return NANOVLLM_GEMM_EINVAL;
    hipLaunchKernelGGL((splitk_lines_kernel<BF, BF, AG, RG, WAVES, LPB>), dim3(static_cast<uint32_t>(blocks)),
                       dim3(WAVES * 64), 0, s, static_cast<const uint16_t*>(p.a), static_cast<const uint16_t*>(p.b),
                       p.c, p.m, p.n, p.k, p.lda, p.ldb, p.ldc);
    return check_launch("splitk_lines");
}


struct SweepConfig {
    int (*launch)(const Problem&, hipStream_t);
    const char* name;
    int max_m;
    int kn;   // 1: B[K,N] (ldb = N), else W[N,K] (ldb = K)
};

#define DECODE_SWEEP_CONFIGS(X) \
    X((launch_cfg<BF, BF, 8, 1, 16, 1, 16, EPI_NONE>), "lds rows=8 rg=16 waves=16 lpb=1", 8, 0) \
    X((launch_cfg<BF, BF, 8, 2, 16, 1, 16, EPI_NONE>), "lds rows=8 rg=32 waves=16 lpb=1", 8, 0) \
    X((launch_cfg<BF, BF, 8, 2, 8, 2, 16, EPI_NONE>), "lds rows=8 rg=32 waves=8 lpb=2", 8, 0) \
    X((launch_cfg<BF, BF, 16, 1, 16, 1, 16, EPI_NONE>), "lds rows=16 rg=16 waves=16 lpb=1", 16, 0) \
    X((launch_cfg<BF, BF, 16, 2, 16, 1, 16, EPI_NONE>), "lds rows=16 rg=32 waves=16 lpb=1", 16, 0) \
    X((launch_cfg<BF, BF, 16, 2, 8, 2, 16, EPI_NONE>), "lds rows=16 rg=32 waves=8 lpb=2", 16, 0) \
    X((launch_cfg<BF, BF, 32, 1, 16, 1, 16, EPI_NONE>), "lds rows=32 rg=16 waves=16 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 32, 2, 16, 1, 16, EPI_NONE>), "lds rows=32 rg=32 waves=16 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 32, 2, 8, 2, 16, EPI_NONE>), "lds rows=32 rg=32 waves=8 lpb=2", 32, 0) \
    X((launch_cfg<BF, BF, 8, 2, 8, 1, 16, EPI_NONE>), "lds rows=8 rg=32 waves=8 lpb=1", 8, 0) \
    X((launch_cfg<BF, BF, 8, 3, 16, 1, 16, EPI_NONE>), "lds rows=8 rg=48 waves=16 lpb=1", 8, 0) \
    X((launch_cfg<BF, BF, 8, 4, 16, 1, 16, EPI_NONE>), "lds rows=8 rg=64 waves=16 lpb=1", 8, 0) \
    X((launch_cfg<BF, BF, 16, 2, 8, 1, 16, EPI_NONE>), "lds rows=16 rg=32 waves=8 lpb=1", 16, 0) \
    X((launch_cfg<BF, BF, 16, 3, 16, 1, 16, EPI_NONE>), "lds rows=16 rg=48 waves=16 lpb=1", 16, 0) \
    X((launch_cfg<BF, BF, 32, 1, 8, 1, 16, EPI_NONE>), "lds rows=32 rg=16 waves=8 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 32, 2, 8, 1, 16, EPI_NONE>), "lds rows=32 rg=32 waves=8 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 8, 2, 16, 1, 16, EPI_NONE, PRO_NONE, 0, 1>), "areg rows=8 rg=32 waves=16 lpb=1", 8, 0) \
    X((launch_cfg<BF, BF, 16, 2, 16, 1, 16, EPI_NONE, PRO_NONE, 0, 1>), "areg rows=16 rg=32 waves=16 lpb=1", 16, 0) \
    X((launch_cfg<BF, BF, 32, 2, 16, 1, 16, EPI_NONE, PRO_NONE, 0, 1>), "areg rows=32 rg=32 waves=16 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 32, 1, 16, 1, 16, EPI_NONE, PRO_NONE, 0, 1>), "areg rows=32 rg=16 waves=16 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 32, 3, 16, 1, 16, EPI_NONE, PRO_NONE, 0, 1>), "areg rows=32 rg=48 waves=16 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 32, 4, 16, 1, 16, EPI_NONE, PRO_NONE, 0, 1>), "areg rows=32 rg=64 waves=16 lpb=1", 32, 0) \
    X((launch_cfg<BF, BF, 32, 2, 8, 2, 16, EPI_NONE, PRO_NONE, 0, 1>), "areg rows=32 rg=32 waves=8 lpb=2", 32, 0) \
    X((launch_cfg<BF, BF, 8, 4, 16, 1, 16, EPI_NONE, PRO_NONE, 1>), "kn rows=8 cols=64 waves=16 lpb=1", 8, 1) \
    X((launch_cfg<BF, BF, 8, 4, 8, 1, 8, EPI_NONE, PRO_NONE, 1>), "kn rows=8 cols=64 waves=8 lpb=1", 8, 1) \
    X((launch_cfg<BF, BF, 16, 4, 8, 1, 8, EPI_NONE, PRO_NONE, 1>), "kn rows=16 cols=64 waves=8 lpb=1", 16, 1) \
    X((launch_cfg<BF, BF, 32, 4, 8, 1, 8, EPI_NONE, PRO_NONE, 1>), "kn rows=32 cols=64 waves=8 lpb=1", 32, 1) \
    X((launch_lines<1, 1, 16, 1>), "lines rows=8 rg=8 waves=16 lpb=1", 8, 0) \
    X((launch_lines<1, 2, 16, 1>), "lines rows=8 rg=16 waves=16 lpb=1", 8, 0) \
    X((launch_lines<1, 4, 16, 1>), "lines rows=8 rg=32 waves=16 lpb=1", 8, 0) \
    X((launch_lines<1, 8, 16, 1>), "lines rows=8 rg=64 waves=16 lpb=1", 8, 0) \
    X((launch_lines<1, 1, 8, 2>), "lines rows=8 rg=8 waves=8 lpb=2", 8, 0) \
    X((launch_lines<1, 2, 8, 2>), "lines rows=8 rg=16 waves=8 lpb=2", 8, 0) \
    X((launch_lines<1, 4, 8, 2>), "lines rows=8 rg=32 waves=8 lpb=2", 8, 0) \
    X((launch_lines<1, 8, 8, 2>), "lines rows=8 rg=64 waves=8 lpb=2", 8, 0) \
    X((launch_lines<1, 1, 4, 4>), "lines rows=8 rg=8 waves=4 lpb=4", 8, 0) \
    X((launch_lines<1, 2, 4, 4>), "lines rows=8 rg=16 waves=4 lpb=4", 8, 0) \
    X((launch_lines<1, 4, 4, 4>), "lines rows=8 rg=32 waves=4 lpb=4", 8, 0) \
    X((launch_lines<2, 1, 16, 1>), "lines rows=16 rg=8 waves=16 lpb=1", 16, 0) \
    X((launch_lines<2, 2, 16, 1>), "lines rows=16 rg=16 waves=16 lpb=1", 16, 0) \
    X((launch_lines<2, 4, 16, 1>), "lines rows=16 rg=32 waves=16 lpb=1", 16, 0) \
    X((launch_lines<2, 1, 8, 2>), "lines rows=16 rg=8 waves=8 lpb=2", 16, 0) \
    X((launch_lines<2, 2, 8, 2>), "lines rows=16 rg=16 waves=8 lpb=2", 16, 0) \
    X((launch_lines<2, 4, 8, 2>), "lines rows=16 rg=32 waves=8 lpb=2", 16, 0) \
    X((launch_lines<2, 8, 8, 2>), "lines rows=16 rg=64 waves=8 lpb=2", 16, 0) \
    X((launch_lines<2, 1, 4, 4>), "lines rows=16 rg=8 waves=4 lpb=4", 16, 0) \
    X((launch_lines<2, 2, 4, 4>), "lines rows=16 rg=16 waves=4 lpb=4", 16, 0) \
    X((launch_lines<2, 4, 4, 4>), "lines rows=16 rg=32 waves=4 lpb=4", 16, 0) \
    X((launch_lines<4, 1, 16, 1>), "lines rows=32 rg=8 waves=16 lpb=1", 32, 0) \
    X((launch_lines<4, 2, 16, 1>), "lines rows=32 rg=16 waves=16 lpb=1", 32, 0) \
    X((launch_lines<4, 4, 16, 1>), "lines rows=32 rg=32 waves=16 lpb=1", 32, 0) \
    X((launch_lines<4, 1, 8, 2>), "lines rows=32 rg=8 waves=8 lpb=2", 32, 0) \
    X((launch_lines<4, 2, 8, 2>), "lines rows=32 rg=16 waves=8 lpb=2", 32, 0) \
    X((launch_lines<4, 4, 8, 2>), "lines rows=32 rg=32 waves=8 lpb=2", 32, 0) \
    X((launch_lines<4, 1, 4, 4>), "lines rows=32 rg=8 waves=4 lpb=4", 32, 0) \
    X((launch_lines<4, 2, 4, 4>), "lines rows=32 rg=16 waves=4 lpb=4", 32, 0) \
    X((launch_cfg<BF, BF, 8, 2, 8, 2, 8, EPI_NONE>), "lds rows=8 rg=32 waves=8 lpb=2 parts=8", 8, 0) \
    X((launch_cfg<BF, BF, 8, 2, 8, 1, 8, EPI_NONE>), "lds rows=8 rg=32 waves=8 lpb=1 parts=8", 8, 0) \
    X((launch_cfg<BF, BF, 8, 4, 8, 1, 8, EPI_NONE>), "lds rows=8 rg=64 waves=8 lpb=1 parts=8", 8, 0) \
    X((launch_cfg<BF, BF, 8, 4, 4, 1, 4, EPI_NONE>), "lds rows=8 rg=64 waves=4 lpb=1 parts=4", 8, 0) \
    X((launch_cfg<BF, BF, 8, 8, 4, 1, 4, EPI_NONE>), "lds rows=8 rg=128 waves=4 lpb=1 parts=4", 8, 0) \
    X((launch_cfg<BF, BF, 8, 2, 4, 2, 4, EPI_NONE>), "lds rows=8 rg=32 waves=4 lpb=2 parts=4", 8, 0) \
    X((launch_cfg<BF, BF, 8, 4, 8, 2, 8, EPI_NONE>), "lds rows=8 rg=64 waves=8 lpb=2 parts=8", 8, 0) \
    X((launch_cfg<BF, BF, 8, 4, 4, 2, 4, EPI_NONE>), "lds rows=8 rg=64 waves=4 lpb=2 parts=4", 8, 0) \
    X((launch_cfg<BF, BF, 8, 8, 4, 2, 4, EPI_NONE>), "lds rows=8 rg=128 waves=4 lpb=2 parts=4", 8, 0) \
    X((launch_cfg<BF, BF, 16, 2, 8, 1, 8, EPI_NONE>), "lds rows=16 rg=32 waves=8 lpb=1 parts=8", 16, 0) \
    X((launch_cfg<BF, BF, 16, 4, 8, 1, 8, EPI_NONE>), "lds rows=16 rg=64 waves=8 lpb=1 parts=8", 16, 0) \
    X((launch_cfg<BF, BF, 16, 4, 4, 1, 4, EPI_NONE>), "lds rows=16 rg=64 waves=4 lpb=1 parts=4", 16, 0) \
    X((launch_cfg<BF, BF, 16, 8, 4, 1, 4, EPI_NONE>), "lds rows=16 rg=128 waves=4 lpb=1 parts=4", 16, 0) \
    X((launch_cfg<BF, BF, 16, 2, 8, 2, 8, EPI_NONE>), "lds rows=16 rg=32 waves=8 lpb=2 parts=8", 16, 0) \
    X((launch_cfg<BF, BF, 16, 4, 4, 2, 4, EPI_NONE>), "lds rows=16 rg=64 waves=4 lpb=2 parts=4", 16, 0) \
    X((launch_cfg<BF, BF, 16, 8, 8, 1, 8, EPI_NONE>), "lds rows=16 rg=128 waves=8 lpb=1 parts=8", 16, 0) \
    X((launch_cfg<BF, BF, 32, 8, 4, 1, 4, EPI_NONE>), "lds rows=32 rg=128 waves=4 lpb=1 parts=4", 32, 0) \
    X((launch_cfg<BF, BF, 32, 4, 4, 1, 4, EPI_NONE>), "lds rows=32 rg=64 waves=4 lpb=1 parts=4", 32, 0) \
    X((launch_cfg<BF, BF, 32, 4, 8, 1, 8, EPI_NONE>), "lds rows=32 rg=64 waves=8 lpb=1 parts=8", 32, 0) \
    X((launch_cfg<BF, BF, 32, 2, 8, 1, 8, EPI_NONE>), "lds rows=32 rg=32 waves=8 lpb=1 parts=8", 32, 0) \
    X((launch_cfg<BF, BF, 32, 4, 4, 2, 4, EPI_NONE>), "lds rows=32 rg=64 waves=4 lpb=2 parts=4", 32, 0) \
    X((launch_cfg<BF, BF, 32, 2, 4, 2, 4, EPI_NONE>), "lds rows=32 rg=32 waves=4 lpb=2 parts=4", 32, 0) \
    X((launch_cfg<BF, BF, 32, 2, 8, 2, 8, EPI_NONE>), "lds rows=32 rg=32 waves=8 lpb=2 parts=8", 32, 0) \
    X((launch_cfg<BF, BF, 32, 6, 4, 1, 4, EPI_NONE>), "lds rows=32 rg=96 waves=4 lpb=1 parts=4", 32, 0)

#define X(fn, name, rows, kn) {fn, name, rows, kn},
const SweepConfig kConfigs[] = {DECODE_SWEEP_CONFIGS(X)};
#undef X
constexpr int kCount = int(sizeof(kConfigs) / sizeof(kConfigs[0]));

}  // namespace
}  // namespace nvg

extern "C" {

int nvsweep_decode_count(void) { return nvg::kCount; }

const char* nvsweep_decode_name(int cfg) { return cfg >= 0 && cfg < nvg::kCount ? nvg::kConfigs[cfg].name : ""; }

int nvsweep_decode_max_m(int cfg) { return cfg >= 0 && cfg < nvg::kCount ? nvg::kConfigs[cfg].max_m : 0; }

// 1 when configuration `cfg` takes B[K,N] (ldb = N), 0 for W[N,K], -1 for a bad index.
int nvsweep_decode_kn(int cfg) { return cfg >= 0 && cfg < nvg::kCount ? nvg::kConfigs[cfg].kn : -1; }

// C[M,N] = A[M,K] W[N,K]^T (or A B with B[K,N] for a B[K,N] configuration)
// in bf16 on configuration `cfg`; -1 for a bad configuration or sizes it
// cannot run (M above its rows, K not a multiple of 8, N not a multiple of
// 8 on B[K,N], null pointers).
int nvsweep_decode(int cfg, const void* a, const void* w, void* c, int64_t m, int64_t n, int64_t k, void* stream) {
    if (cfg < 0 || cfg >= nvg::kCount) return -1;
    if (a == nullptr || w == nullptr || c == nullptr) return -1;
    if (m < 1 || m > nvg::kConfigs[cfg].max_m || n < 1 || k < 8 || k % 8 != 0) return -1;
    const bool kn = nvg::kConfigs[cfg].kn != 0;
    if (kn && (n < 8 || n % 8 != 0)) return -1;
    nvg::Problem p{};
    p.a = a;
    p.b = w;
    p.c = c;
    p.m = m;
    p.n = n;
    p.k = k;
    p.lda = k;
    p.ldb = kn ? n : k;
    p.ldc = n;
    p.b_layout = kn ? NANOVLLM_GEMM_B_KN : NANOVLLM_GEMM_B_NK;
    p.dtype_in = NANOVLLM_GEMM_BF16;
    p.dtype_out = NANOVLLM_GEMM_BF16;
    return nvg::kConfigs[cfg].launch(p, static_cast<hipStream_t>(stream)) == NANOVLLM_GEMM_OK ? 0 : -1;
}

}  // extern "C"
