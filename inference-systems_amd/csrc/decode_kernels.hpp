// Kernels of splitk_decode (the launch table is in gemm_decode.hip), shared
// with the configuration sweep library (decode_sweep.hip).
#pragma once
#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kLine = 64;   // K elements per line: 128 bytes = 8 chunks of 16 bytes

// Source of the K-tail chunks: 16 zero bytes in global memory.
__device__ u32x4_t g_decode_zero = {0u, 0u, 0u, 0u};

// 16-byte load through a global-address-space pointer (a generic pointer that
// may also hold the zero chunk's address would otherwise make it a flat load,
// which also counts on the LDS counter).
__device__ __forceinline__ u32x4_t load16_global(const void* p) {
    typedef const __attribute__((address_space(1))) u32x4_t* gptr;
    return *reinterpret_cast<gptr>(reinterpret_cast<uintptr_t>(p));
}

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

// B[K,N] lines: position of column chunk c of k-row r is c ^ kn_line_swizzle(r).
// A fragment read touches k-rows {0..3, 8..11, 16..19, 24..27} (+ 4) x 32
// bytes; rows r and r + 2 share banks (128-byte rows), and flipping chunk
// pairs by bits 1 and 3 of r puts the 8 rows of each parity on 4 distinct
// 32-byte bank groups, two each: two clocks, the minimum for 512 bytes.
__device__ __forceinline__ int kn_line_swizzle(int r) { return 2 * (((r >> 1) & 1) | ((r >> 2) & 2)); }

// Whether a splitk_decode configuration builds: its LDS (the copy regions
// and, with the norm prologue, the per-wave sums of squares) within the
// 160 KiB of a CU, the partition tiles within a wave's region, the copies
// of a batch within the vmcnt range.  Mirrors the kernel's declarations.
constexpr int64_t kLdsBytes = 160 * 1024;

template <int AROWS, int RG, int WAVES, int LPB, int PARTS, int PRO>
constexpr bool decode_cfg_fits() {
    constexpr int MG = AROWS == 8 ? 1 : AROWS / 16;
    constexpr int IA = AROWS / 8;
    constexpr int IL = 2 * RG + IA + (PRO == PRO_NONE ? 0 : IA);
    constexpr int REGION = LPB * IL * 64;
    constexpr int PW = PARTS / WAVES;
    constexpr int64_t lds = int64_t(WAVES) * REGION * 16 + (PRO == PRO_ADD_NORM ? WAVES : 1) * MG * 16 * 4;
    return lds <= kLdsBytes && PW * RG * MG * 256 <= 4 * REGION && LPB * IL < 64 && PARTS % WAVES == 0;
}

// RG groups of 16 W rows per workgroup, AROWS rows of A copied per line
// (8, 16, 32 or 64: M rounded up), WAVES waves splitting K, LPB lines per wave
// in flight at once, PARTS K partitions (a multiple of WAVES), PRO the
// prologue on A.
//
// KN: B is given as B[K,N] (row stride ldb >= N, N a multiple of 8), the
// reference bench's layout, with RG = 4: a workgroup takes 64 output
// columns, and a line is 64 k-rows of B x those 64 columns (128 bytes of a
// k-row), copied as they lie by 8 instructions of 8 k-rows.  k-row r holds
// its 16-byte column chunks in position chunk ^ kn_line_swizzle(r), and the
// W fragments (8 consecutive k of one column per lane) are read back with
// gfx950's transposing LDS read, two ds_read_b64_tr_b16 of 4 k-rows each.
template <int DT, int DT_OUT, int AROWS, int RG, int WAVES, int LPB, int PARTS, int EPI, int PRO, int KN = 0,
          int AREG = 0>
__global__ __launch_bounds__(WAVES * 64) void splitk_decode_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ w, void* __restrict__ c,
    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, uint64_t* __restrict__ keys,
    ProArgs pro, SampleArgs sa) {
    static_assert(AROWS == 8 || AROWS == 16 || AROWS == 32 || AROWS == 64, "rows of A per line");
    constexpr int MG = AROWS == 8 ? 1 : AROWS / 16;   // 16-row groups of A in the MFMA
    constexpr int IW = 2 * RG;                 // W copies per line (8 rows each)
    // AREG: A's fragments are loaded from global memory straight into
    // registers (with the line's W copies), so only W passes through LDS.
    static_assert(!AREG || (PRO == PRO_NONE && !KN), "register A: plain A, W[N,K]");
    constexpr int IA = AREG ? 0 : AROWS / 8;   // A copies per line
    constexpr int IP = PRO == PRO_NONE ? 0 : IA;   // gate or residual copies per line
    constexpr int IL = IW + IA + IP;
    static_assert(PRO == PRO_NONE || EPI == EPI_NONE || (PRO == PRO_ADD_NORM && EPI == EPI_SILU_MUL),
                  "prologues come with the plain store (and the norm also with SiLU-and-mul)");
    static_assert(!KN || (RG == 4 && EPI == EPI_NONE && PRO == PRO_NONE), "B[K,N]: 64 columns, plain store");
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
        if constexpr (KN) {
            // k-row 8 h + r8 of the line; column chunks past N read the last
            // chunk (their outputs are not stored).
            const int kr = 8 * h + r8;
            const int64_t col = n0 + 8 * ((lane & 7) ^ kn_line_swizzle(kr));
            wsrc[h] = w + int64_t(kr) * ldb + min_i64(col, n - 8);
        } else if constexpr (EPI == EPI_SILU_MUL) {
            wsrc[h] = w + ((r & 1) ? n : 0) * ldb + min_i64(n0 + 16 * (r >> 1) + rr, n - 1) * ldb + chunk * 8;
        } else {
            wsrc[h] = w + min_i64(n0 + 16 * r + rr, n - 1) * ldb + chunk * 8;
        }
    }
    const uint16_t* asrc[IA > 0 ? IA : 1];
#pragma unroll
    for (int h = 0; h < IA; ++h) asrc[h] = a + min_i64(8 * h + r8, m - 1) * lda + chunk * 8;
    // AREG: lane l's A fragment of group g is row 16 g + l % 16 (rows 0-7
    // twice at AROWS = 8), 8 elements at chunk l / 16 of each 32-wide K-step.
    const uint16_t* afrag[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g)
        afrag[g] = a + min_i64(AROWS == 8 ? (lane & 7) : 16 * g + (lane & 15), m - 1) * lda + 8 * (lane >> 4);
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

    // EPI_ARGMAX: thread x ranks row x / ETPR of A.  On a sampled head the
    // noise of its columns (log2 E, which does not depend on the logits) is
    // drawn while the first lines' copies are in flight, for every row (a
    // greedy row's draws go unused), so a sampled row costs the epilogue
    // little more than a greedy one.  With 4 or more columns a thread (QUAD)
    // it takes groups of 4 adjacent columns, 4 (x % ETPR) + 4 ETPR i + j, one
    // draw serving 4; with fewer it takes columns x % ETPR + ETPR i, as the
    // greedy ranking does, one draw each.  The row's temperature is
    // requested before any copy and first used in the epilogue, when every
    // copy has landed.
    constexpr int EROWS = MG * 16;
    constexpr int ETPR = WAVES * 64 / EROWS;
    static_assert(EPI != EPI_ARGMAX || (ETPR >= 1 && ETPR <= 64 && (ETPR & (ETPR - 1)) == 0),
                  "a row's threads share a wave");
    constexpr int ECOLS = 16 * RG;
    constexpr bool QUAD = ECOLS >= 4 * ETPR;
    constexpr int NIT = EPI != EPI_ARGMAX ? 1 : QUAD ? (ECOLS + 4 * ETPR - 1) / (4 * ETPR) : (ECOLS + ETPR - 1) / ETPR;
    const int erow = threadIdx.x / ETPR, esub = threadIdx.x % ETPR;
    // One unconditional global load (rows past M read row M - 1; a greedy
    // head reads the first 4 bytes of A, unused), so no branch joins on the
    // loaded register before its use, and it is counted on vmcnt alone.
    float traw = 0.0f;   // the row's temperature as given
    float nlog[NIT][QUAD ? 4 : 1];
    if constexpr (EPI == EPI_ARGMAX) {
        const float* tp = sa.temperature != nullptr ? sa.temperature + min_i64(erow, m - 1)
                                                    : reinterpret_cast<const float*>(a);
        traw = *tp;
    }
    // The empty asm statements take every draw, so the draws stay ahead of
    // the wait for the copies that follows them.
    auto draw_noise = [&]() {
        if (sa.temperature == nullptr) return;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            if constexpr (QUAD) {
                const int c4 = 4 * esub + 4 * ETPR * it;
                const u32x4_t x = sample_words(erow, (n0 + c4) >> 2, sa);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    nlog[it][j] = gumbel_log2e(x[j]);
                    asm volatile("" : "+v"(nlog[it][j]));
                }
            } else {
                // Column cc's word is word cc % 4 of its quad (n0 is a
                // multiple of 16).
                const int cc = esub + ETPR * it;
                const u32x4_t x = sample_words(erow, (n0 + cc) >> 2, sa);
                const int j = cc & 3;
                nlog[it][0] = gumbel_log2e(j == 0 ? x[0] : j == 1 ? x[1] : j == 2 ? x[2] : x[3]);
                asm volatile("" : "+v"(nlog[it][0]));
            }
        }
    };
    bool drawn = false;

    // Wave w takes lines w + WAVES j, j = 0, 1, ...: line j of a trip goes to
    // partition w + WAVES (j % PW), in batches of LPB copied together.
    for (int64_t l0 = wave; l0 < lines; l0 += int64_t(WAVES) * ROUND) {
#pragma unroll
        for (int bt = 0; bt < ROUND / LPB; ++bt) {
            if (l0 + int64_t(WAVES) * (bt * LPB) >= lines) break;
            u32x4_t nwv[LPB][2];   // PRO_ADD_NORM: the norm weight at the lane's two fragment chunks
            u32x4_t areg[LPB][2][MG];   // AREG: the lane's A fragments of each K-step
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
                if constexpr (KN) {
                    // k-rows past K and A chunks past K copy zeros.
                    const bool in_k = koff + chunk * 8 < k;
#pragma unroll
                    for (int h = 0; h < IW; ++h)
                        dma16_stream(koff + 8 * h + r8 < k ? static_cast<const void*>(wsrc[h] + koff * ldb) : zero,
                                     dst + 1024u * h);
#pragma unroll
                    for (int h = 0; h < IA; ++h)
                        dma16(in_k ? static_cast<const void*>(asrc[h] + koff) : zero, dst + 1024u * (IW + h));
                } else if (koff + kLine <= k) {
#pragma unroll
                    for (int h = 0; h < IW; ++h) dma16_stream(wsrc[h] + koff, dst + 1024u * h);
#pragma unroll
                    for (int h = 0; h < IA; ++h) dma16(asrc[h] + koff, dst + 1024u * (IW + h));
#pragma unroll
                    for (int h = 0; h < IP; ++h) dma16(psrc[h] + pk, dst + 1024u * (IW + IA + h));
                } else {
                    // K tail (K % 8 == 0): chunks past K copy zeros into W and A.
                    const bool in_k = koff + chunk * 8 < k;
#pragma unroll
                    for (int h = 0; h < IW; ++h)
                        dma16_stream(in_k ? static_cast<const void*>(wsrc[h] + koff) : zero, dst + 1024u * h);
#pragma unroll
                    for (int h = 0; h < IA; ++h)
                        dma16(in_k ? static_cast<const void*>(asrc[h] + koff) : zero, dst + 1024u * (IW + h));
#pragma unroll
                    for (int h = 0; h < IP; ++h)
                        dma16(in_k ? static_cast<const void*>(psrc[h] + pk) : zero, dst + 1024u * (IW + IA + h));
                }
                if constexpr (AREG) {
                    if (koff + kLine <= k) {
#pragma unroll
                        for (int st = 0; st < 2; ++st)
#pragma unroll
                            for (int g = 0; g < MG; ++g) areg[t][st][g] = load16_global(afrag[g] + koff + 32 * st);
                    } else {
                        // K tail: chunks past K load the zero chunk (a
                        // pointer select, so no wait is tied to the value).
#pragma unroll
                        for (int st = 0; st < 2; ++st) {
                            const bool in_k = koff + (4 * st + grp) * 8 < k;
#pragma unroll
                            for (int g = 0; g < MG; ++g)
                                areg[t][st][g] =
                                    load16_global(in_k ? static_cast<const void*>(afrag[g] + koff + 32 * st) : zero);
                        }
                    }
                }
            }
            if constexpr (EPI == EPI_ARGMAX) {
                if (!drawn) {
                    draw_noise();
                    drawn = true;
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
                    if constexpr (KN) {
                        // Lane 16 g + j of a read points at k-row 32 st + 8 g + j / 4
                        // (+ 4 for the second) and columns 16 r + 4 (j % 4) .. + 3; lane
                        // 16 g + i receives k = 32 st + 8 g .. + 7 of column 16 r + i.
                        typedef short v4i16_t __attribute__((ext_vector_type(4)));
                        typedef __attribute__((address_space(3))) v4i16_t* lds_v4;
                        const int kr = 32 * st + 8 * grp + (i16 >> 2);
                        const uint32_t rowb = lds_address(lb) + uint32_t(kr) * 128u + 8u * (i16 & 1);
#pragma unroll
                        for (int r = 0; r < RG; ++r) {
                            const int ch = (2 * r + ((i16 & 3) >> 1)) ^ kn_line_swizzle(kr);
                            const uint32_t a0 = rowb + uint32_t(ch) * 16u;
                            const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4)(uintptr_t)a0);
                            const v4i16_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4)(uintptr_t)(a0 + 512u));
                            const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi4);
                            wf[r] = u32x4_t{l2[0], l2[1], h2[0], h2[1]};
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < RG; ++r) wf[r] = lb[(2 * r + hi) * 64 + slot];
                    }
#pragma unroll
                    for (int g = 0; g < MG; ++g)
                        af[g] = AREG ? areg[t][st][g] : lb[(IW + (AROWS == 8 ? 0 : 2 * g + hi)) * 64 + slot];
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
    if constexpr (EPI == EPI_ARGMAX) {
        if (!drawn) draw_noise();   // a wave with no line of K
    }

    // acc[q][r][g][v] is D[n = 4*(l/16) + v][m = l%16] of W-row group r,
    // A-row group g, in partition wave + WAVES q.  Each wave writes its
    // partition tiles to its own region (its last reads of it completed at
    // the wait above); partition p then sits in wave p % WAVES, slot
    // p / WAVES.  Within a 16 x 16 tile, (n, m) is stored at
    // 64 (n % 4) + 16 (n / 4) + (m ^ 4 (n % 4)), i.e. in bank
    // 16 (n / 4) + (m ^ 4 (n % 4)) of the 64: one write instruction (fixed
    // v, lanes over n / 4 and m) and the reads below (a wave's threads over
    // 16 n and 4 consecutive m) each touch 64 distinct banks.  (With
    // 16 n + (m ^ n) the writes touched 16 banks, four lanes each: the
    // bank-conflict stalls the counters showed.)
    auto part = [&](int wv, int q, int r, int g, int nn, int mm) -> float& {
        return reinterpret_cast<float*>(&buf[wv][0])[((q * RG + r) * MG + g) * 256 + 64 * (nn & 3) + 16 * (nn >> 2) +
                                                     (mm ^ (4 * (nn & 3)))];
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
        constexpr int TPR = ETPR;
        const int row = erow, sub = esub;
        uint64_t best = 0;
        const float t = sa.temperature != nullptr && row < m && traw > 1e-10f ? traw : 0.0f;   // 0: greedy
        if (row < m && t == 0.0f) {
            for (int cc = sub; cc < 16 * RG; cc += TPR) {
                if (n0 + cc >= n) break;
                const uint64_t key = argmax_key(ranked_logit(total(cc >> 4, row >> 4, cc & 15, row & 15), sa), n0 + cc);
                best = key > best ? key : best;
            }
        } else if (row < m) {
            // A sampled row, its columns assigned as the draws made during
            // the K loop were.
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                if constexpr (QUAD) {
                    const int c4 = 4 * sub + 4 * TPR * it;
                    if (c4 >= ECOLS || n0 + c4 >= n) break;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int cc = c4 + j;
                        if (n0 + cc >= n) break;
                        const float v = gumbel_apply(ranked_logit(total(cc >> 4, row >> 4, cc & 15, row & 15), sa),
                                                     t, nlog[it][j]);
                        const uint64_t key = argmax_key(v, n0 + cc);
                        best = key > best ? key : best;
                    }
                } else {
                    const int cc = sub + TPR * it;
                    if (cc >= ECOLS || n0 + cc >= n) break;
                    const float v = gumbel_apply(ranked_logit(total(cc >> 4, row >> 4, cc & 15, row & 15), sa), t,
                                                 nlog[it][0]);
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

template <int DT, int DT_OUT, int AROWS, int RG, int WAVES, int LPB, int PARTS, int EPI, int PRO = PRO_NONE,
          int KN = 0, int AREG = 0>
int launch_cfg(const Problem& p, hipStream_t s) {
    constexpr int OG = EPI == EPI_SILU_MUL ? RG / 2 : RG;
    if (p.m > AROWS) return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "splitk_decode: M above the configuration's rows");
    const int64_t blocks = (p.n + 16 * OG - 1) / (16 * OG);
    if (blocks > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "splitk_decode: grid too large");
    const dim3 grid(static_cast<uint32_t>(blocks)), block(WAVES * 64);
    if (EPI == EPI_ARGMAX) *p.key_blocks = blocks;
    const ProArgs pro{static_cast<const uint16_t*>(p.a2), p.lda2, p.group, p.group_stride,
                      static_cast<const uint16_t*>(p.norm_w), p.eps, static_cast<uint16_t*>(p.res_out), p.ldres};
    hipLaunchKernelGGL((splitk_decode_kernel<DT, DT_OUT, AROWS, RG, WAVES, LPB, PARTS, EPI, PRO, KN, AREG>), grid, block, 0, s,
                       static_cast<const uint16_t*>(p.a), static_cast<const uint16_t*>(p.b), p.c, p.m, p.n, p.k,
                       p.lda, p.ldb, p.ldc, p.keys, pro, p.sample);
    return check_launch("splitk_decode");
}

}  // namespace
}  // namespace nvg
