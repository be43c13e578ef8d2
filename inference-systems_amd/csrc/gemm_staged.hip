// mfma_staged: the prefill GEMM for gfx950, C[M,N] = A[M,K] * W[N,K]^T with
// BF16/FP16 inputs, fp32 accumulation and a bf16/fp16/fp32 epilogue.
//
// This is the "staged" rung of the reference ladder
// (cuda_kernels/gemm/src/gemm_bench.cu:117-196, gemm_wmma.cu:116-207)
// designed for CDNA4 instead of translated:
//   * BM x BN macro tile per 256-thread workgroup (4 waves in a 2x2 grid),
//     K-tiles of 64 elements;
//   * v_mfma_f32_32x32x16_{bf16,f16} with W as the first operand and A as
//     the second, so each lane ends with 4 consecutive output columns per
//     accumulator quad and stores them with one 8- or 16-byte write;
//   * 16-byte coalesced global loads (8 threads cover one 128-byte row
//     segment), register-staged into a double-buffered LDS tile;
//   * LDS rows of 64 elements are 8 chunks of 16 bytes; chunk c of row r
//     sits at position c ^ (r & 7), so both the ds_write_b128 of a row
//     segment and the ds_read_b128 of an MFMA fragment (8 consecutive rows,
//     one chunk) touch 8 distinct 16-byte bank groups;
//   * one barrier per K-tile, the next tile's global loads in flight while
//     the current one is multiplied;
//   * XCD-aware tile order so the tiles that share A and W rows run on the
//     same XCD's L2.
// Rows past M or N are clamped for loading and masked at the store; the K
// tail is zero-filled per 8-element chunk (K must be a multiple of 8).
#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kBK = 64;        // K elements per tile = 8 chunks of 16 bytes
constexpr int kChunks = kBK / 8;

template <int DT, int DT_OUT, int BM, int BN>
__global__ __launch_bounds__(256) void mfma_staged_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc,
    int tiles_m, int tiles_n, int c_vec) {
    constexpr int WM = BM / 2;           // wave tile rows (M)
    constexpr int WN = BN / 2;           // wave tile cols (N)
    constexpr int MJ = WM / 32;          // 32-row blocks of A per wave
    constexpr int NI = WN / 32;          // 32-row blocks of W per wave
    constexpr int A_PER = BM * kChunks / 256;
    constexpr int B_PER = BN * kChunks / 256;
    static_assert(A_PER * 256 == BM * kChunks && B_PER * 256 == BN * kChunks, "tile / thread mismatch");

    __shared__ u32x4_t lds[2][(BM + BN) * kChunks];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int half = lane >> 5;
    const int r32 = lane & 31;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 8, tm, tn);
    const int64_t m0 = int64_t(tm) * BM;
    const int64_t n0 = int64_t(tn) * BN;

    // Global -> LDS assignment: chunk e = tid + 256 r is row e / 8, chunk e % 8.
    const int my_chunk = tid & 7;
    const uint16_t* a_src[A_PER];
    const uint16_t* w_src[B_PER];
    int a_dst[A_PER], w_dst[B_PER];
#pragma unroll
    for (int r = 0; r < A_PER; ++r) {
        const int row = (tid >> 3) + 32 * r;
        const int64_t gm = min(m0 + row, m - 1);
        a_src[r] = a + gm * lda + my_chunk * 8;
        a_dst[r] = row * kChunks + (my_chunk ^ (row & 7));
    }
#pragma unroll
    for (int r = 0; r < B_PER; ++r) {
        const int row = (tid >> 3) + 32 * r;
        const int64_t gn = min(n0 + row, n - 1);
        w_src[r] = w + gn * ldb + my_chunk * 8;
        w_dst[r] = BM * kChunks + row * kChunks + (my_chunk ^ (row & 7));
    }

    u32x4_t ra[A_PER], rb[B_PER];
    auto load_tile = [&](int64_t k0) {
        const bool full = k0 + kBK <= k;
        const bool in_k = k0 + my_chunk * 8 < k;
#pragma unroll
        for (int r = 0; r < A_PER; ++r)
            ra[r] = (full || in_k) ? load16(a_src[r] + k0) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int r = 0; r < B_PER; ++r)
            rb[r] = (full || in_k) ? load16(w_src[r] + k0) : u32x4_t{0u, 0u, 0u, 0u};
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int r = 0; r < A_PER; ++r) lds[buf][a_dst[r]] = ra[r];
#pragma unroll
        for (int r = 0; r < B_PER; ++r) lds[buf][w_dst[r]] = rb[r];
    };

    f32x16_t acc[NI][MJ];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j] = f32x16_t{};

    // Fragment rows: lane l reads row (base + l % 32); since every base is a
    // multiple of 32, the swizzle key (row & 7) is (l & 7).
    const int swz = lane & 7;
    const int a_row0 = wm * WM + r32;
    const int w_row0 = BM + wn * WN + r32;

    const int64_t ktiles = (k + kBK - 1) / kBK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int64_t t = 0; t < ktiles; ++t) {
        const int cur = int(t & 1);
        const bool more = t + 1 < ktiles;
        if (more) load_tile((t + 1) * kBK);
        const u32x4_t* tile = lds[cur];
#pragma unroll
        for (int kk = 0; kk < kChunks / 2; ++kk) {
            const int chunk = (2 * kk + half) ^ swz;
            u32x4_t af[MJ], wf[NI];
#pragma unroll
            for (int j = 0; j < MJ; ++j) af[j] = tile[(a_row0 + 32 * j) * kChunks + chunk];
#pragma unroll
            for (int i = 0; i < NI; ++i) wf[i] = tile[(w_row0 + 32 * i) * kChunks + chunk];
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int j = 0; j < MJ; ++j) acc[i][j] = mfma_32x32x16<DT>(wf[i], af[j], acc[i][j]);
        }
        if (more) store_tile(cur ^ 1);
        __syncthreads();
    }

    // Epilogue.  acc[i][j][v] is D[n][m] with n = 8 (v/4) + 4 half + v%4 and
    // m = l % 32 inside the (i, j) block, so each quad v/4 is 4 consecutive
    // columns of one output row.
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int64_t row = m0 + wm * WM + 32 * j + r32;
        if (row >= m) continue;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t col = n0 + wn * WN + 32 * i + 8 * q + 4 * half;
                const f32x16_t& v = acc[i][j];
                const float x0 = v[4 * q], x1 = v[4 * q + 1], x2 = v[4 * q + 2], x3 = v[4 * q + 3];
                const int64_t idx = row * ldc + col;
                if (c_vec && col + 3 < n) {
                    if constexpr (DT_OUT == NANOVLLM_GEMM_F32) {
                        *reinterpret_cast<f32x4_t*>(static_cast<float*>(c) + idx) = f32x4_t{x0, x1, x2, x3};
                    } else {
                        uint32_t lo, hi;
                        if constexpr (DT_OUT == NANOVLLM_GEMM_BF16) {
                            lo = f32_to_bf16_rne(x0) | (uint32_t(f32_to_bf16_rne(x1)) << 16);
                            hi = f32_to_bf16_rne(x2) | (uint32_t(f32_to_bf16_rne(x3)) << 16);
                        } else {
                            lo = f32_to_f16_rne(x0) | (uint32_t(f32_to_f16_rne(x1)) << 16);
                            hi = f32_to_f16_rne(x2) | (uint32_t(f32_to_f16_rne(x3)) << 16);
                        }
                        *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(c) + idx) = u32x2_t{lo, hi};
                    }
                } else {
                    if (col < n) store_elem<DT_OUT>(c, idx, x0);
                    if (col + 1 < n) store_elem<DT_OUT>(c, idx + 1, x1);
                    if (col + 2 < n) store_elem<DT_OUT>(c, idx + 2, x2);
                    if (col + 3 < n) store_elem<DT_OUT>(c, idx + 3, x3);
                }
            }
        }
    }
}

// Tile shape for a problem: the largest tile that still gives at least
// one workgroup per CU (256 CUs), else the smallest.
struct TileChoice {
    int bm, bn;
};

TileChoice choose_tile(int64_t m, int64_t n) {
    auto tiles = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
    if (tiles(128, 256) >= 256) return {128, 256};
    if (tiles(256, 128) >= 256 && m >= 256) return {256, 128};
    return {128, 128};
}

template <int DT, int DT_OUT, int BM, int BN>
int launch_tile(const Problem& p, hipStream_t s) {
    const int64_t tiles_m = (p.m + BM - 1) / BM, tiles_n = (p.n + BN - 1) / BN;
    if (tiles_m * tiles_n > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "mfma_staged: grid too large");
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n)), block(256);
    const int out_bytes = DT_OUT == NANOVLLM_GEMM_F32 ? 4 : 2;
    // Vector stores write 4 elements: 16 B (fp32) or 8 B (bf16/fp16).
    const int c_vec = (reinterpret_cast<uintptr_t>(p.c) % (4 * out_bytes) == 0) && (p.ldc % 4 == 0);
    hipLaunchKernelGGL((mfma_staged_kernel<DT, DT_OUT, BM, BN>), grid, block, 0, s,
                       static_cast<const uint16_t*>(p.a), static_cast<const uint16_t*>(p.b), p.c,
                       p.m, p.n, p.k, p.lda, p.ldb, p.ldc, int(tiles_m), int(tiles_n), c_vec);
    return check_launch("mfma_staged");
}

template <int DT, int DT_OUT>
int launch_typed(const Problem& p, hipStream_t s) {
    const TileChoice t = choose_tile(p.m, p.n);
    if (t.bm == 128 && t.bn == 256) return launch_tile<DT, DT_OUT, 128, 256>(p, s);
    if (t.bm == 256 && t.bn == 128) return launch_tile<DT, DT_OUT, 256, 128>(p, s);
    return launch_tile<DT, DT_OUT, 128, 128>(p, s);
}

}  // namespace

int launch_mfma_staged(const Problem& p, hipStream_t s) {
    if (p.dtype_in == NANOVLLM_GEMM_BF16) {
        if (p.dtype_out == NANOVLLM_GEMM_BF16) return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_BF16>(p, s);
        return launch_typed<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_F32>(p, s);
    }
    if (p.dtype_out == NANOVLLM_GEMM_F16) return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F16>(p, s);
    return launch_typed<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F32>(p, s);
}

}  // namespace nvg
