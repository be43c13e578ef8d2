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
#include "decode_kernels.hpp"

namespace nvg {
namespace {

// Configurations measured on MI355X.  AROWS is M rounded up to 8, 16, 32 or
// 64; "rows" counts the W rows read (2 N for SiLU-and-mul).
//   * rows < 65536: 32 W rows per 16-wave workgroup, one line per wave, so
//     all 16 lines of K = 1024 are in flight at once, while those
//     workgroups fit the CUs at one each (larger N: launch_rows); N = 6144, K = 1024,
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

constexpr int64_t kDecodeCus = 256;

// Workgroups of a configuration resident on one CU at once (LDS, waves and
// registers), from the runtime's occupancy query, once per configuration.
// The query enqueues nothing (it may run under graph capture); should it
// fail, one workgroup per CU is assumed and the error is cleared so the
// launch that follows does not report it.
template <int DT, int DT_OUT, int AROWS, int RG, int WAVES, int EPI, int PRO>
int64_t resident_per_cu() {
    static const int64_t per_cu = [] {
        int blocks = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &blocks, reinterpret_cast<const void*>(&splitk_decode_kernel<DT, DT_OUT, AROWS, RG, WAVES, 1, 16, EPI, PRO>),
            WAVES * 64, 0);
        if (e != hipSuccess) (void)hipGetLastError();
        return int64_t(e == hipSuccess && blocks > 0 ? blocks : 1);
    }();
    return per_cu;
}

// Candidate (RG, WAVES) of the wide-W choice, one line per wave in flight,
// 16 K partitions; those whose LDS does not fit are skipped at compile time.
struct RowsChoice {
    int64_t busiest = INT64_MAX, rounds = 0, grid = 0;
    int waves = 0, id = -1;
    bool better_than(const RowsChoice& o) const {
        if (busiest != o.busiest) return busiest < o.busiest;
        if (rounds != o.rounds) return rounds < o.rounds;
        if (grid != o.grid) return grid < o.grid;
        return waves > o.waves;
    }
};

template <int DT, int DT_OUT, int EPI, int AROWS, int PRO, int RG, int WAVES>
void consider(RowsChoice& best, int id, int64_t rows) {
    if constexpr (decode_cfg_fits<AROWS, RG, WAVES, 1, 16, PRO>()) {
        RowsChoice c;
        c.grid = (rows + 16 * RG - 1) / (16 * RG);
        c.busiest = (c.grid + kDecodeCus - 1) / kDecodeCus * 16 * RG;
        const int64_t slots = kDecodeCus * resident_per_cu<DT, DT_OUT, AROWS, RG, WAVES, EPI, PRO>();
        c.rounds = (c.grid + slots - 1) / slots;
        c.waves = WAVES;
        c.id = id;
        if (c.better_than(best)) best = c;
    }
}

template <int DT, int DT_OUT, int EPI, int AROWS, int PRO, int RG, int WAVES>
int launch_if(int id, int want, const Problem& p, hipStream_t s) {
    if constexpr (decode_cfg_fits<AROWS, RG, WAVES, 1, 16, PRO>())
        if (id == want) return launch_cfg<DT, DT_OUT, AROWS, RG, WAVES, 1, 16, EPI, PRO>(p, s);
    return 1;   // not this candidate
}

template <int DT, int DT_OUT, int EPI, int AROWS, int PRO>
int launch_picked(const Problem& p, hipStream_t s, int64_t rows) {
    RowsChoice best;
    consider<DT, DT_OUT, EPI, AROWS, PRO, 2, 16>(best, 0, rows);
    consider<DT, DT_OUT, EPI, AROWS, PRO, 3, 16>(best, 1, rows);
    consider<DT, DT_OUT, EPI, AROWS, PRO, 1, 16>(best, 2, rows);
    consider<DT, DT_OUT, EPI, AROWS, PRO, 2, 8>(best, 3, rows);
    consider<DT, DT_OUT, EPI, AROWS, PRO, 3, 8>(best, 4, rows);
    consider<DT, DT_OUT, EPI, AROWS, PRO, 1, 8>(best, 5, rows);
    int rc = 1;
    if (rc == 1) rc = launch_if<DT, DT_OUT, EPI, AROWS, PRO, 2, 16>(0, best.id, p, s);
    if (rc == 1) rc = launch_if<DT, DT_OUT, EPI, AROWS, PRO, 3, 16>(1, best.id, p, s);
    if (rc == 1) rc = launch_if<DT, DT_OUT, EPI, AROWS, PRO, 1, 16>(2, best.id, p, s);
    if (rc == 1) rc = launch_if<DT, DT_OUT, EPI, AROWS, PRO, 2, 8>(3, best.id, p, s);
    if (rc == 1) rc = launch_if<DT, DT_OUT, EPI, AROWS, PRO, 3, 8>(4, best.id, p, s);
    if (rc == 1) rc = launch_if<DT, DT_OUT, EPI, AROWS, PRO, 1, 8>(5, best.id, p, s);
    if (rc == 1) return set_error(NANOVLLM_GEMM_ELAUNCH, "splitk_decode: no configuration fits");
    return rc;
}

template <int DT, int DT_OUT, int EPI, int AROWS, int PRO>
int launch_rows(const Problem& p, hipStream_t s) {
    const int64_t rows = EPI == EPI_SILU_MUL ? 2 * p.n : p.n;
    if (rows >= kWideN) {
        // M = 1 takes the configuration of M = 2-8, so rows of M = 1-16 share
        // one sum order.  A kernel of its own for M = 1 (16 W rows per 4-wave
        // workgroup, fragments loaded straight into registers, eight loads per
        // lane in flight) led until W was copied non-temporally; against this
        // configuration after that (W over two copies, three interleaved runs)
        // it took 54.8-56.4 against 50.4-51.2 us for fp32 logits, 53.4-55.2
        // against 52.3-53.0 for the greedy head and 52.0-52.3 against
        // 50.8-51.2 for the sampled one, and was removed.
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
    // Above 2048 rows (plain store, LM-head epilogues, prologues): 32 W rows
    // per 16-wave workgroup while those workgroups fit the 256 CUs at one
    // each (every line of a 1024-wide K in flight at once); on wider W the
    // configuration whose busiest CU streams the fewest W rows, then the one
    // that needs the fewest rounds of resident workgroups, then the fewest
    // workgroups (see pick_rows).  A grid one workgroup past a round pays
    // for a second one.  Measured on MI355X (W streamed from HBM, bench.py
    // --decode-sweep), M = 4 / 8 / 16 / 32: N = 8224 (257 workgroups of 32
    // rows) 5.74 / 5.91 / 7.31 / 8.45 us with 32 rows throughout, 5.31 /
    // 5.44 / 5.68 us with 48 rows and 7.43 us with 8-wave workgroups of 16
    // rows three to a CU at M = 32; N = 16384, M = 16 / 32: 9.13 / 10.20
    // against 8.04 / 8.95 us with 8-wave workgroups of 32 rows resident
    // three / two to a CU.
    if constexpr (EPI != EPI_SILU_MUL) {
        if ((rows + 31) / 32 > kDecodeCus) return launch_picked<DT, DT_OUT, EPI, AROWS, PRO>(p, s, rows);
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

// B[K,N] (the reference bench's layout), plain store, M <= 64: 64 columns
// per workgroup, K split over the waves by 64-k-row lines; 16 waves up to
// M = 8 (144 KiB of LDS), 8 waves with 8 K partitions above.
template <int DT, int DT_OUT>
int launch_kn(const Problem& p, hipStream_t s) {
    if (p.m <= 8) return launch_cfg<DT, DT_OUT, 8, 4, 16, 1, 16, EPI_NONE, PRO_NONE, 1>(p, s);
    if (p.m <= 16) return launch_cfg<DT, DT_OUT, 16, 4, 8, 1, 8, EPI_NONE, PRO_NONE, 1>(p, s);
    if (p.m <= 32) return launch_cfg<DT, DT_OUT, 32, 4, 8, 1, 8, EPI_NONE, PRO_NONE, 1>(p, s);
    if (p.m <= 64) return launch_cfg<DT, DT_OUT, 64, 4, 8, 1, 8, EPI_NONE, PRO_NONE, 1>(p, s);
    return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "splitk_decode: B[K,N] above M = 64");
}

}  // namespace

int launch_splitk_decode(const Problem& p, hipStream_t s) {
    if (p.b_layout == NANOVLLM_GEMM_B_KN) {
        if (p.epi != EPI_NONE || p.pro != PRO_NONE)
            return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "splitk_decode: B[K,N] takes the plain GEMM only");
        if (p.dtype_in == NANOVLLM_GEMM_BF16) {
            if (p.dtype_out == NANOVLLM_GEMM_BF16) return launch_kn<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_BF16>(p, s);
            return launch_kn<NANOVLLM_GEMM_BF16, NANOVLLM_GEMM_F32>(p, s);
        }
        if (p.dtype_out == NANOVLLM_GEMM_F16) return launch_kn<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F16>(p, s);
        return launch_kn<NANOVLLM_GEMM_F16, NANOVLLM_GEMM_F32>(p, s);
    }
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
