// splitk_decode: the bandwidth-bound small-M GEMM (M <= 32, and the plain
// GEMM up to M = 64), C = A * W^T with W[N,K] in the nn.Linear layout.  At
// these shapes the work is streaming W once from HBM (N*K*2 bytes) while A
// (M*K*2 bytes) stays in L2.  Design:
//   * one workgroup per 16 * RG rows of W; its waves split K, taking
//     64-element lines (128 bytes of a row) round robin, LPB lines at a time;
//   * W and A reach LDS by global_load_lds_dwordx4 in whole 128-byte lines:
//     one instruction copies one line of each of 8 rows.  The MFMA fragment
//     layout (lane l holds row l % 16) would have each load instruction touch
//     16 rows x 64 bytes; on MI355X a load instruction costs by the cache
//     lines it touches, and a 12.6 MB W streamed as whole lines takes
//     ~0.8 us less than as half lines (4.05 against 4.85 us, same grid);
//   * lane L of a copy writes LDS slot L, row L / 8, and fetches chunk
//     (L % 8) ^ (L / 8) of its row's line, so a fragment read (16 rows, one
//     chunk) hits 8 distinct 16-byte slots in every group of 8 lanes;
//   * each wave reads back only what it copied (no barrier in the K loop),
//     v_mfma_f32_16x16x32 with W as the first operand (16 rows of W) and up
//     to two 16-row groups of A as the second; rows of A past M repeat row
//     M - 1 and their outputs are not stored;
//   * line L is accumulated into K partition L % PARTS, each wave owning
//     PARTS / WAVES partitions, and the partition sums are added in LDS in
//     partition order (deterministic, no atomics, no workspace) and written
//     once.  The order of every sum depends on PARTS alone, so all
//     configurations with PARTS = 16 (every W of fewer than 65536 rows)
//     give bit-identical results for a given row of A and row of W, whatever
//     N: a merged projection equals its separate parts.
// It replaces the reference's cuBLAS fallback for decode shapes and the
// M == 16 direct-WMMA special case (cuda_kernels/gemm/src/gemm_bench.cu:260-273).
#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kLine = 64;   // K elements per line: 128 bytes = 8 chunks of 16 bytes

// Source of the K-tail chunks: 16 zero bytes in global memory.
__device__ u32x4_t g_decode_zero = {0u, 0u, 0u, 0u};

// Operands of the prologues (PRO_GATE, PRO_ADD_NORM; see gemm_common.hpp).
struct ProArgs {
    const uint16_t* a2;      // gate or residual, leading dimension lda2
    int64_t lda2;
    int64_t group, group_stride;   // PRO_GATE: k -> (k / group) * group_stride + k % group
    const uint16_t* norm_w;  // PRO_ADD_NORM: [K] zero-centred weight
    float eps;
    uint16_t* res_out;       // PRO_ADD_NORM: round(h + r), leading dimension ldres
    int64_t ldres;
};

// RG groups of 16 W rows per workgroup, AROWS rows of A copied per line
// (8, 16, 32 or 64: M rounded up), WAVES waves splitting K, LPB lines per wave
// in flight at once, PARTS K partitions (a multiple of WAVES), PRO the
// prologue on A.
template <int DT, int DT_OUT, int AROWS, int RG, int WAVES, int LPB, int PARTS, int EPI, int PRO>
__global__ __launch_bounds__(WAVES * 64) void splitk_decode_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, uint64_t* __restrict__ keys,
    ProArgs pro, SampleArgs sa) {
    static_assert(AROWS == 8 || AROWS == 16 || AROWS == 32 || AROWS == 64, "rows of A per line");
    constexpr int MG = AROWS == 8 ? 1 : AROWS / 16;   // 16-row groups of A in the MFMA
    constexpr int IW = 2 * RG;                 // W copies per line (8 rows each)
    constexpr int IA = AROWS / 8;              // A copies per line
    constexpr int IP = PRO == PRO_NONE ? 0 : IA;   // gate or residual copies per line
    constexpr int IL = IW + IA + IP;
    static_assert(PRO == PRO_NONE || EPI == EPI_NONE || (PRO == PRO_ADD_NORM && EPI == EPI_SILU_MUL),
                  "prologues come with the plain store (and the norm also with SiLU-and-mul)");
    static_assert(LPB * IL < 64, "vmcnt range");
    static_assert(PARTS % WAVES == 0, "whole partitions per wave");
    constexpr int PW = PARTS / WAVES;                  // partitions per wave
    constexpr int ROUND = LPB > PW ? LPB : PW;         // lines per wave per loop trip
    static_assert(ROUND % LPB == 0 && ROUND % PW == 0, "copy batches and partitions tile a trip");
    // Per wave: LPB lines x IL copies x 64 lanes x 16 bytes.  After the K
    // loop a wave's region holds its partition sums for the final addition.
    constexpr int REGION = LPB * IL * 64;
    static_assert(PW * RG * MG * 256 <= 4 * REGION, "partition tiles fit in a wave's region");
    __shared__ u32x4_t buf[WAVES][REGION];
    // PRO_ADD_NORM: per wave, the sum of s^2 over its lines, per row of A.
    __shared__ float sspart[PRO == PRO_ADD_NORM ? WAVES : 1][MG * 16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i16 = lane & 15;   // fragment row (W: first operand, A: second)
    const int grp = lane >> 4;   // fragment chunk within the 32-wide K-step
    const int r8 = lane >> 3;    // copy: row within the instruction's 8
    const int chunk = (lane & 7) ^ r8;   // copy: chunk of the line this lane fetches

    // EPI_SILU_MUL: W-row groups pair up, group 2s holding gate rows and
    // group 2s + 1 the up rows of the same 16 output columns.
    static_assert(EPI != EPI_SILU_MUL || RG % 2 == 0, "gate/up group pairs");
    constexpr int OG = EPI == EPI_SILU_MUL ? RG / 2 : RG;   // 16-column output groups per workgroup
    // Consecutive column blocks go to consecutive workgroups, which the
    // hardware hands to the 8 XCDs round robin.  Giving each XCD a contiguous
    // run of blocks instead (xcd_remap, so the two workgroups writing one
    // 128-byte output line share an L2) measured 0.3 us slower on every
    // decode shape (N = 6144, K = 1024, M = 1-64; 1024 x 3584): W streams
    // better when each XCD's reads spread over the whole matrix.
    const int64_t n0 = int64_t(blockIdx.x) * 16 * OG;         // first output column
    const uint16_t* wsrc[IW];
#pragma unroll
    for (int h = 0; h < IW; ++h) {
        const int r = h >> 1;
        const int64_t rr = 8 * (h & 1) + r8;
        if constexpr (EPI == EPI_SILU_MUL)
            wsrc[h] = w + ((r & 1) ? n : 0) * ldb + min_i64(n0 + 16 * (r >> 1) + rr, n - 1) * ldb + chunk * 8;
        else
            wsrc[h] = w + min_i64(n0 + 16 * r + rr, n - 1) * ldb + chunk * 8;
    }
    const uint16_t* asrc[IA];
#pragma unroll
    for (int h = 0; h < IA; ++h) asrc[h] = a + min_i64(8 * h + r8, m - 1) * lda + chunk * 8;
    const uint16_t* psrc[IP > 0 ? IP : 1];
#pragma unroll
    for (int h = 0; h < IP; ++h) psrc[h] = pro.a2 + min_i64(8 * h + r8, m - 1) * pro.lda2 + chunk * 8;
    const void* zero = &g_decode_zero;
    asm volatile("" : "+s"(zero));

    // Fragment slots: row i16 of a 16-row group sits in copy 2 g + i16 / 8,
    // slot 8 (i16 % 8) + (chunk ^ (i16 % 8)), for chunk grp (first 32-wide
    // K-step of the line) and 4 + grp (second).
    const int x = i16 & 7, hi = i16 >> 3;
    const int slot0 = 8 * x + (grp ^ x), slot1 = 8 * x + ((4 + grp) ^ x);

    const int64_t lines = (k + kLine - 1) / kLine;
    const uint32_t base = lds_address(&buf[wave][0]);
    f32x4_t acc[PW][RG][MG];
    // PRO_ADD_NORM: this lane's sum of s^2 for its fragment rows.
    float ss[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) ss[g] = 0.0f;
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int r = 0; r < RG; ++r)
#pragma unroll
            for (int g = 0; g < MG; ++g) acc[q][r][g] = f32x4_t{};

    // Wave w takes lines w + WAVES j, j = 0, 1, ...: line j of a trip goes to
    // partition w + WAVES (j % PW), in batches of LPB copied together.
    for (int64_t l0 = wave; l0 < lines; l0 += int64_t(WAVES) * ROUND) {
#pragma unroll
        for (int bt = 0; bt < ROUND / LPB; ++bt) {
            if (l0 + int64_t(WAVES) * (bt * LPB) >= lines) break;
            u32x4_t nwv[LPB][2];   // PRO_ADD_NORM: the norm weight at the lane's two fragment chunks
#pragma unroll
            for (int t = 0; t < LPB; ++t) {
                const int64_t line = l0 + int64_t(WAVES) * (bt * LPB + t);
                if (line >= lines) break;
                const uint32_t dst = base + uint32_t(t * IL) * 1024u;
                const int64_t koff = line * kLine;
                // PRO_GATE: a line never straddles a gate group (group % 64 == 0).
                int64_t pk = koff;
                if constexpr (PRO == PRO_GATE) pk = (koff / pro.group) * pro.group_stride + koff % pro.group;
                if constexpr (PRO == PRO_ADD_NORM) {
#pragma unroll
                    for (int st = 0; st < 2; ++st)
                        nwv[t][st] = load16(pro.norm_w + min_i64(koff + (4 * st + grp) * 8, k - 8));
                }
                if (koff + kLine <= k) {
#pragma unroll
                    for (int h = 0; h < IW; ++h) dma16(wsrc[h] + koff, dst + 1024u * h);
#pragma unroll
                    for (int h = 0; h < IA; ++h) dma16(asrc[h] + koff, dst + 1024u * (IW + h));
#pragma unroll
                    for (int h = 0; h < IP; ++h) dma16(psrc[h] + pk, dst + 1024u * (IW + IA + h));
                } else {
                    // K tail (K % 8 == 0): chunks past K copy zeros into W and A.
                    const bool in_k = koff + chunk * 8 < k;
#pragma unroll
                    for (int h = 0; h < IW; ++h)
                        dma16(in_k ? static_cast<const void*>(wsrc[h] + koff) : zero, dst + 1024u * h);
#pragma unroll
                    for (int h = 0; h < IA; ++h)
                        dma16(in_k ? static_cast<const void*>(asrc[h] + koff) : zero, dst + 1024u * (IW + h));
#pragma unroll
                    for (int h = 0; h < IP; ++h)
                        dma16(in_k ? static_cast<const void*>(psrc[h] + pk) : zero, dst + 1024u * (IW + IA + h));
                }
            }
            wait_vmcnt<0>();
            if constexpr (PRO == PRO_GATE) {
                // The gate, in place on this batch's copies of A: lane j takes
                // column j of each line for the M real rows only (the copy's
                // rows past M repeat row M - 1 and their outputs are not
                // stored), so the work per lane is M sigmoids a line (against
                // 16 per lane on fragments at M <= 8).  Row r sits in copy
                // r / 8 at 16-bit position 8 (8 (r % 8) + ((j / 8) ^ (r % 8))) + j % 8.
#pragma unroll
                for (int t = 0; t < LPB; ++t) {
                    const int64_t line = l0 + int64_t(WAVES) * (bt * LPB + t);
                    if (line >= lines) break;
                    uint16_t* lh = reinterpret_cast<uint16_t*>(&buf[wave][t * IL * 64]);
                    for (int r = 0; r < AROWS; ++r) {
                        if (r >= m) break;
                        const int r8v = r & 7;
                        const int pos = 8 * (8 * r8v + ((lane >> 3) ^ r8v)) + (lane & 7);
                        uint16_t* ap = lh + (IW + (r >> 3)) * 512 + pos;
                        *ap = gate1<DT>(*ap, lh[(IW + IA + (r >> 3)) * 512 + pos]);
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < LPB; ++t) {
                const int64_t line = l0 + int64_t(WAVES) * (bt * LPB + t);
                if (line >= lines) break;
                const int q = (bt * LPB + t) % PW;   // compile-time after unrolling
                const u32x4_t* lb = &buf[wave][t * IL * 64];
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const int slot = st ? slot1 : slot0;
                    u32x4_t wf[RG], af[MG];
#pragma unroll
                    for (int r = 0; r < RG; ++r) wf[r] = lb[(2 * r + hi) * 64 + slot];
#pragma unroll
                    for (int g = 0; g < MG; ++g) af[g] = lb[(IW + (AROWS == 8 ? 0 : 2 * g + hi)) * 64 + slot];
                    if constexpr (PRO == PRO_ADD_NORM) {
                        // Element k of this fragment chunk; chunks past K are zero in h and r.
                        const int64_t kc = line * kLine + (4 * st + grp) * 8;
                        const bool in_k = kc < k;
                        const u32x4_t wv = in_k ? nwv[t][st] : u32x4_t{0u, 0u, 0u, 0u};
                        // Every workgroup forms s for all of A; line L's new residual is
                        // written by workgroup L mod gridDim.x.
                        const bool writes =
                            __builtin_amdgcn_readfirstlane(int(uint32_t(line) % gridDim.x)) == int(blockIdx.x);
#pragma unroll
                        for (int g = 0; g < MG; ++g) {
                            u32x4_t res;
                            af[g] = add_norm8<DT>(af[g], lb[(IW + IA + (AROWS == 8 ? 0 : 2 * g + hi)) * 64 + slot],
                                                  wv, ss[g], res);
                            // each element once: rows 8..15 of an 8-row copy repeat rows 0..7
                            const int64_t row = 16 * g + i16;
                            if (writes && in_k && row < m && (AROWS != 8 || i16 < 8))
                                *reinterpret_cast<u32x4_t*>(pro.res_out + row * pro.ldres + kc) = res;
                        }
                    }
#pragma unroll
                    for (int r = 0; r < RG; ++r)
#pragma unroll
                        for (int g = 0; g < MG; ++g)
                            acc[q][r][g] = mfma_16x16x32<DT>(wf[r], af[g], acc[q][r][g]);
                }
            }
            // The next lines' copies overwrite the slots just read.
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
    }

    // acc[q][r][g][v] is D[n = 4*(l/16) + v][m = l%16] of W-row group r,
    // A-row group g, in partition wave + WAVES q.  Each wave writes its
    // partition tiles to its own region (its last reads of it completed at
    // the wait above); partition p then sits in wave p % WAVES, slot
    // p / WAVES.  Within a 16 x 16 tile, (n, m) is stored at 16 n + (m ^ n):
    // the writes (16 lanes along m) and the reads below (16 lanes along n)
    // both hit 16 distinct banks.
    auto part = [&](int wv, int q, int r, int g, int nn, int mm) -> float& {
        return reinterpret_cast<float*>(&buf[wv][0])[(((q * RG + r) * MG + g) * 16 + nn) * 16 + (mm ^ nn)];
    };
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int r = 0; r < RG; ++r)
#pragma unroll
            for (int g = 0; g < MG; ++g)
#pragma unroll
                for (int v = 0; v < 4; ++v) part(wave, q, r, g, 4 * grp + v, i16) = acc[q][r][g][v];
    if constexpr (PRO == PRO_ADD_NORM) {
        // The wave's sum of s^2 per row: its 4 lanes of a row (one per
        // fragment chunk) added by a butterfly, the same sum in every lane.
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            float v = ss[g];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (grp == 0) sspart[wave][16 * g + i16] = v;
        }
    }
    __syncthreads();
    // Sum of the partitions in partition order.
    auto total = [&](int r, int g, int nn, int mm) {
        float sum = part(0, 0, r, g, nn, mm);
#pragma unroll
        for (int pp = 1; pp < PARTS; ++pp) sum += part(pp % WAVES, pp / WAVES, r, g, nn, mm);
        return sum;
    };

    if constexpr (EPI == EPI_ARGMAX) {
        // Per row of A, the best of this workgroup's 16 * RG columns: TPR
        // adjacent threads per row each take every TPR-th column, then a
        // butterfly over those lanes (keys order by value, then by lowest
        // column, so the result does not depend on the split).
        constexpr int ROWS = MG * 16;
        constexpr int TPR = WAVES * 64 / ROWS;
        static_assert(TPR >= 1 && TPR <= 64 && (TPR & (TPR - 1)) == 0, "a row's threads share a wave");
        const int row = threadIdx.x / TPR, sub = threadIdx.x % TPR;
        uint64_t best = 0;
        const float t = row < m ? sample_temperature(row, sa) : 0.0f;
        if (row < m && t == 0.0f) {
            for (int cc = sub; cc < 16 * RG; cc += TPR) {
                if (n0 + cc >= n) break;
                const uint64_t key = argmax_key(ranked_logit(total(cc >> 4, row >> 4, cc & 15, row & 15), sa), n0 + cc);
                best = key > best ? key : best;
            }
        } else if (row < m) {
            // A sampled row: groups of 4 adjacent columns, so one noise draw
            // serves 4 scores (n0 is a multiple of 16).
            for (int c4 = 4 * sub; c4 < 16 * RG; c4 += 4 * TPR) {
                if (n0 + c4 >= n) break;
                const u32x4_t x = sample_words(row, (n0 + c4) >> 2, sa);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int cc = c4 + j;
                    if (n0 + cc >= n) break;
                    const float v = gumbel_score(ranked_logit(total(cc >> 4, row >> 4, cc & 15, row & 15), sa), t, x[j]);
                    const uint64_t key = argmax_key(v, n0 + cc);
                    best = key > best ? key : best;
                }
            }
        }
#pragma unroll
        for (int off = TPR / 2; off >= 1; off >>= 1) {
            const uint64_t other = (uint64_t(uint32_t(__shfl_xor(int(best >> 32), off))) << 32) |
                                   uint64_t(uint32_t(__shfl_xor(int(best & 0xFFFFFFFFu), off)));
            best = other > best ? other : best;
        }
        if (sub == 0 && row < m) keys[row * int64_t(gridDim.x) + blockIdx.x] = best;
        return;
    }

    for (int e = threadIdx.x; e < OG * MG * 256; e += WAVES * 64) {
        const int o = e / (MG * 256);
        const int g = (e / 256) % MG;
        const int nn = e & 15;
        const int mm = (e >> 4) & 15;
        const int64_t row = g * 16 + mm;
        const int64_t col = n0 + 16 * o + nn;
        if (row >= m || col >= n) continue;
        // PRO_ADD_NORM: the row's scale, from the waves' sums of s^2 in wave order.
        float rs = 1.0f;
        if constexpr (PRO == PRO_ADD_NORM) {
            float sum_sq = sspart[0][row];
#pragma unroll
            for (int wv = 1; wv < WAVES; ++wv) sum_sq += sspart[wv][row];
            rs = norm_scale(sum_sq, k, pro.eps);
        }
        if constexpr (EPI == EPI_SILU_MUL) {
            float gate = total(2 * o, g, nn, mm), up = total(2 * o + 1, g, nn, mm);
            if constexpr (PRO == PRO_ADD_NORM) {
                gate *= rs;
                up *= rs;
            }
            store_elem<DT_OUT>(c, row * ldc + col, silu_f32(gate) * up);
        } else if constexpr (PRO == PRO_ADD_NORM) {
            store_elem<DT_OUT>(c, row * ldc + col, total(o, g, nn, mm) * rs);
        } else {
            store_elem<DT_OUT>(c, row * ldc + col, total(o, g, nn, mm));
        }
    }
}

// M = 1 on very wide W (the LM head): 16 W rows per 4-wave workgroup, the
// MFMA fragments loaded straight into registers, eight 16-byte loads per
// lane in flight.  Its loads touch 16 half-lines each, but with ~9500
// workgroups at full occupancy it keeps more bytes in flight than the
// LDS-staged kernel can (N = 151936: 48.4 us, 80% of HBM, against 50.9 us
// for the best LDS-staged configuration).  EPI_NONE or EPI_ARGMAX.
constexpr int kRegWaves = 4, kRegUnroll = 8, kRegStep = 32;

template <int DT, int DT_OUT, int EPI>
__global__ __launch_bounds__(kRegWaves * 64) void splitk_regs_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, uint64_t* __restrict__ keys,
    SampleArgs sa) {
    static_assert(EPI != EPI_SILU_MUL, "gate/up pairs need the LDS-staged kernel");
    __shared__ float red[kRegWaves][16][16];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i16 = lane & 15;
    const int grp = lane >> 4;
    const int64_t n0 = int64_t(blockIdx.x) * 16;
    const uint16_t* wp = w + min_i64(n0 + i16, n - 1) * ldb + grp * 8;
    const bool a_in = i16 < m;
    const uint16_t* ap = a + (a_in ? i16 : 0) * lda + grp * 8;
    const int64_t steps = (k + kRegStep - 1) / kRegStep;
    f32x4_t acc = f32x4_t{};
    for (int64_t s0 = wave; s0 < steps; s0 += kRegWaves * kRegUnroll) {
        u32x4_t wf[kRegUnroll], af[kRegUnroll];
#pragma unroll
        for (int u = 0; u < kRegUnroll; ++u) {
            const int64_t ks = (s0 + kRegWaves * u) * kRegStep;
            const bool in_k = ks + grp * 8 < k;   // K % 8 == 0: a chunk is all in or all out
            wf[u] = in_k ? load16(wp + ks) : u32x4_t{0u, 0u, 0u, 0u};
            af[u] = (in_k && a_in) ? load16(ap + ks) : u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kRegUnroll; ++u) acc = mfma_16x16x32<DT>(wf[u], af[u], acc);
    }
    // acc[v] is D[n = 4 (l / 16) + v][m = l % 16].
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][4 * grp + v][i16] = acc[v];
    __syncthreads();
    // One thread per (column nn, row mm) of the 16 x 16 tile.
    const int nn = threadIdx.x & 15, mm = threadIdx.x >> 4;
    float sum = red[0][nn][mm];
#pragma unroll
    for (int wv = 1; wv < kRegWaves; ++wv) sum += red[wv][nn][mm];
    if constexpr (EPI == EPI_ARGMAX) {
        // Per row of A, the best of the workgroup's 16 columns: a 16-lane
        // max over the keys of one row (lanes 16 mm .. 16 mm + 15).
        uint64_t best = n0 + nn < n && mm < m ? argmax_key(sample_score(sum, mm, n0 + nn, sa), n0 + nn) : 0;
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) {
            const uint64_t other = (uint64_t(uint32_t(__shfl_xor(int(best >> 32), off))) << 32) |
                                   uint64_t(uint32_t(__shfl_xor(int(best & 0xFFFFFFFFu), off)));
            best = other > best ? other : best;
        }
        if (nn == 0 && mm < m) keys[mm * int64_t(gridDim.x) + blockIdx.x] = best;
    } else {
        if (mm < m && n0 + nn < n) store_elem<DT_OUT>(c, mm * ldc + n0 + nn, sum);
    }
}

template <int DT, int DT_OUT, int EPI>
int launch_regs(const Problem& p, hipStream_t s) {
    if (p.m > 16) return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "splitk_decode: M above the configuration's rows");
    const int64_t blocks = (p.n + 15) / 16;
    if (blocks > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "splitk_decode: grid too large");
    if (EPI == EPI_ARGMAX) *p.key_blocks = blocks;
    hipLaunchKernelGGL((splitk_regs_kernel<DT, DT_OUT, EPI>), dim3(static_cast<uint32_t>(blocks)),
                       dim3(kRegWaves * 64), 0, s, static_cast<const uint16_t*>(p.a),
                       static_cast<const uint16_t*>(p.b), p.c, p.m, p.n, p.k, p.lda, p.ldb, p.ldc, p.keys, p.sample);
    return check_launch("splitk_decode");
}

template <int DT, int DT_OUT, int AROWS, int RG, int WAVES, int LPB, int PARTS, int EPI, int PRO = PRO_NONE>
int launch_cfg(const Problem& p, hipStream_t s) {
    constexpr int OG = EPI == EPI_SILU_MUL ? RG / 2 : RG;
    if (p.m > AROWS) return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "splitk_decode: M above the configuration's rows");
    const int64_t blocks = (p.n + 16 * OG - 1) / (16 * OG);
    if (blocks > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "splitk_decode: grid too large");
    const dim3 grid(static_cast<uint32_t>(blocks)), block(WAVES * 64);
    if (EPI == EPI_ARGMAX) *p.key_blocks = blocks;
    const ProArgs pro{static_cast<const uint16_t*>(p.a2), p.lda2, p.group, p.group_stride,
                      static_cast<const uint16_t*>(p.norm_w), p.eps, static_cast<uint16_t*>(p.res_out), p.ldres};
    hipLaunchKernelGGL((splitk_decode_kernel<DT, DT_OUT, AROWS, RG, WAVES, LPB, PARTS, EPI, PRO>), grid, block, 0, s,
                       static_cast<const uint16_t*>(p.a), static_cast<const uint16_t*>(p.b), p.c, p.m, p.n, p.k,
                       p.lda, p.ldb, p.ldc, p.keys, pro, p.sample);
    return check_launch("splitk_decode");
}

// Configurations measured on MI355X.  AROWS is M rounded up to 8, 16, 32 or
// 64; "rows" counts the W rows read (2 N for SiLU-and-mul).
//   * rows < 65536: 32 W rows per 16-wave workgroup, one line per wave, so
//     all 16 lines of K = 1024 are in flight at once; N = 6144, K = 1024,
//     W streamed from HBM, M = 4 / 8 / 16 / 32: 4.54 / 4.57 / 4.81 / 5.58 us
//     against 4.72 / 4.76 / 4.94 / 5.75 us with 8 waves of two lines each
//     (and 5.42 / 5.87 / 7.25 us for the register-loading kernel at M = 8 /
//     16 / 32).  The same W read by a plain streaming kernel takes 3.55 us,
//     and these copies alone 4.01 us (M = 8) / 4.58 us (M = 32); an empty
//     kernel costs 1.56 us per graph node.  With at most 2048 rows (N = 1024, K = 3584,
//     the down and output projections) 16 rows per workgroup give twice the
//     workgroups, with 16 waves along K up to M = 16 (M = 1 / 16 / 32: 4.7 /
//     6.6 / 8.5 us, against 7.0 / 9.0 / 11.7 us with 32 rows).
//   * rows >= 65536 (the LM head, N = 151936, K = 1024): M = 1 runs the
//     register-loading kernel (48.4 us; with a prologue, the M <= 8
//     configuration); M = 8 / 16 / 32: 53.5 / 57.5 / 63.9 us (61.2 / 65.7 /
//     75.8 us with register loading).
//   * 33 <= M <= 64 (the plain GEMM only, below 65536 rows): A's copies now
//     outweigh W's, so 8 waves and 8 K partitions in every configuration,
//     16 / 32 / 48 rows per workgroup up to 4096 / 8192 / 65535 rows.
//     Against mfma_staged, whose 64 x 64 tiles leave most CUs idle on these
//     grids (bf16, M = 64, K = 1024 unless given): N = 1024 3.6 against
//     5.9 us, 1024 x K 3584 6.5 / 15.5, 2048 x K 2048 4.8 / 9.7, 3584 3.8 /
//     6.0, 4096 x K 4096 10.0 / 19.0, 6144 4.6 / 6.0, 8224 5.7 / 6.2; from
//     16384 rows mfma_staged's larger grid wins (7.1 against 9.9 us), and
//     the selection table sends M > 32 there.
// A prologue adds its own copies per line to the same configurations.
constexpr int64_t kWideN = 65536;

// 33 <= M <= 64 below 65536 rows: the plain GEMM, and SiLU-and-mul on
// gate/up row-group pairs (32 rows per workgroup).
template <int DT, int DT_OUT, int EPI>
int launch_rows64(const Problem& p, hipStream_t s) {
    const int64_t rows = EPI == EPI_SILU_MUL ? 2 * p.n : p.n;
    if (rows >= kWideN) return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "splitk_decode: M > 32 needs N < 65536");
    if constexpr (EPI == EPI_SILU_MUL) {
        return launch_cfg<DT, DT_OUT, 64, 2, 8, 1, 8, EPI>(p, s);
    } else {
        if (rows <= 4096) return launch_cfg<DT, DT_OUT, 64, 1, 8, 1, 8, EPI>(p, s);
        if (rows <= 8192) return launch_cfg<DT, DT_OUT, 64, 2, 8, 1, 8, EPI>(p, s);
        return launch_cfg<DT, DT_OUT, 64, 3, 8, 1, 8, EPI>(p, s);
    }
}

template <int DT, int DT_OUT, int EPI, int AROWS, int PRO>
int launch_rows(const Problem& p, hipStream_t s) {
    const int64_t rows = EPI == EPI_SILU_MUL ? 2 * p.n : p.n;
    if (rows >= kWideN) {
        if constexpr (EPI != EPI_SILU_MUL && PRO == PRO_NONE && AROWS == 8)
            if (p.m == 1) return launch_regs<DT, DT_OUT, EPI>(p, s);
        if constexpr (AROWS == 32) return launch_cfg<DT, DT_OUT, 32, 8, 4, 1, 4, EPI, PRO>(p, s);
        else if constexpr (AROWS == 16) return launch_cfg<DT, DT_OUT, 16, 2, 8, 1, 8, EPI, PRO>(p, s);
        else return launch_cfg<DT, DT_OUT, 8, 2, 8, 2, 8, EPI, PRO>(p, s);
    }
    if constexpr (EPI != EPI_SILU_MUL) {
        if (rows <= 2048) {
            if constexpr (AROWS == 32) return launch_cfg<DT, DT_OUT, 32, 1, 8, 1, 16, EPI, PRO>(p, s);
            else return launch_cfg<DT, DT_OUT, AROWS, 1, 16, 1, 16, EPI, PRO>(p, s);
        }
    }
    // 16 waves, one line each: every line of a 1024-wide K is in flight at
    // once.  With 32 rows of A and a prologue operand the copies need 192 KiB
    // of LDS, so that case keeps 8 waves of two lines.
    if constexpr (PRO == PRO_NONE || AROWS <= 16) return launch_cfg<DT, DT_OUT, AROWS, 2, 16, 1, 16, EPI, PRO>(p, s);
    else return launch_cfg<DT, DT_OUT, AROWS, 2, 8, 1, 16, EPI, PRO>(p, s);
}

template <int DT, int DT_OUT, int EPI, int PRO = PRO_NONE>
int launch_epi(const Problem& p, hipStream_t s) {
    if (p.m <= 8) return launch_rows<DT, DT_OUT, EPI, 8, PRO>(p, s);
    if (p.m <= 16) return launch_rows<DT, DT_OUT, EPI, 16, PRO>(p, s);
    if (p.m <= 32) return launch_rows<DT, DT_OUT, EPI, 32, PRO>(p, s);
    if constexpr ((EPI == EPI_NONE || EPI == EPI_SILU_MUL) && PRO == PRO_NONE)
        if (p.m <= 64) return launch_rows64<DT, DT_OUT, EPI>(p, s);
    return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "splitk_decode: M above its limit");
}

template <int DT, int DT_OUT>
int launch_typed(const Problem& p, hipStream_t s) {
    if (p.epi == EPI_SILU_MUL) {
        if (p.pro == PRO_ADD_NORM) return launch_epi<DT, DT_OUT, EPI_SILU_MUL, PRO_ADD_NORM>(p, s);
        return launch_epi<DT, DT_OUT, EPI_SILU_MUL>(p, s);
    }
    if (p.pro == PRO_GATE) return launch_epi<DT, DT_OUT, EPI_NONE, PRO_GATE>(p, s);
    if (p.pro == PRO_ADD_NORM) return launch_epi<DT, DT_OUT, EPI_NONE, PRO_ADD_NORM>(p, s);
    return launch_epi<DT, DT_OUT, EPI_NONE>(p, s);
}

// Greedy LM head: the plain configurations, writing partial keys instead of
// the fp32 logits.
template <int DT>
int launch_argmax(const Problem& p, hipStream_t s) {
    return launch_epi<DT, NANOVLLM_GEMM_F32, EPI_ARGMAX>(p, s);
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
