// Shared definitions for the gfx950 GEMM kernels: problem descriptor,
// element conversions, MFMA wrappers and the launcher declarations that
// capi.cpp dispatches to.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nanovllm_gemm.h"

namespace nvg {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Output epilogues.  EPI_NONE stores the product.  EPI_SILU_MUL is the fused
// SiluAndMul of a gate/up projection: W = [W_gate; W_up] has 2n rows, output
// column j is silu(a . W_gate[j]) * (a . W_up[j]), computed in fp32 from the
// fp32 accumulators and rounded once.
// EPI_ARGMAX is the greedy token of an LM head: no output matrix; each
// workgroup writes, per row of A, one 64-bit key (argmax_key) of the best
// column it computed into a workspace of [M, workgroups along N] keys,
// reduced by launch_argmax_finalize.
constexpr int EPI_NONE = 0;
constexpr int EPI_SILU_MUL = 1;
constexpr int EPI_ARGMAX = 2;

// Prologues on A.  PRO_GATE is the gated-attention output gate: A is used as
// a * sigmoid(g), the sigmoid rounded to the element type and the product
// rounded again (the reference's two element-type tensor ops).  PRO_ADD_NORM
// is the residual add and zero-centred RMSNorm in front of a projection: with
// s = h + r in fp32, the GEMM runs on y = round(s * (1 + w)) and output row i
// is scaled by rsqrt(mean_k s[i][k]^2 + eps) after the sum; round(s) is the
// new residual.
constexpr int PRO_NONE = 0;
constexpr int PRO_GATE = 1;
constexpr int PRO_ADD_NORM = 2;

// Per-row temperatures and noise of the sampled LM head (see sample_score),
// and the type whose rounding of each logit the LM head ranks.
struct SampleArgs {
    const float* temperature = nullptr;   // [M]; nullptr: every row greedy
    uint64_t seed = 0;
    uint64_t offset = 0;
    // NANOVLLM_GEMM_F32: the fp32 accumulator itself.  NANOVLLM_GEMM_BF16 /
    // NANOVLLM_GEMM_F16: the logit rounded (nearest even) to that type, which
    // is what F.linear in the model dtype hands to the sampler
    // (nanovllm/layers/embed_head.py:61, nanovllm/layers/sampler.py:15).
    int logit_dtype = NANOVLLM_GEMM_F32;
};

// One GEMM problem as it crosses the C ABI (see include/nanovllm_gemm.h).
struct Problem {
    const void* a;
    const void* b;
    void* c;
    int64_t m, n, k;
    int64_t lda, ldb, ldc;
    int b_layout;
    int dtype_in;
    int dtype_out;
    int epi = EPI_NONE;   // EPI_SILU_MUL: n output columns from 2n rows of b
    uint64_t* keys = nullptr;         // EPI_ARGMAX: [m, workgroups along N] partial keys
    int64_t* key_blocks = nullptr;    // EPI_ARGMAX: set by the launcher to its workgroups along N
    SampleArgs sample;                // EPI_ARGMAX: per-row temperatures and noise (sampled LM head)
    const float* row_scale = nullptr; // mfma_staged, EPI_NONE / EPI_SILU_MUL: output row i (both
                                      // sums of a SiLU pair) times row_scale[i] before rounding
    int pro = PRO_NONE;
    // PRO_GATE: gate element (i, k) at a2[i * lda2 + (k / group) * group_stride + k % group].
    // PRO_ADD_NORM: residual r[i, k] at a2[i * lda2 + k]; norm weight norm_w[k];
    // the new residual round(h + r) goes to res_out[i * ldres + k].
    const void* a2 = nullptr;
    int64_t lda2 = 0;
    int64_t group = 0, group_stride = 0;
    const void* norm_w = nullptr;
    float eps = 0.0f;
    void* res_out = nullptr;
    int64_t ldres = 0;
};

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Element conversions.  bf16 and fp16 travel as raw 16-bit patterns.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, uint32_t(h) << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return float(__builtin_bit_cast(_Float16, h));
}

template <int DT>
__device__ __forceinline__ float half_to_f32(uint16_t h) {
    if constexpr (DT == NANOVLLM_GEMM_BF16) return bf16_to_f32(h);
    else return f16_to_f32(h);
}

// fp32 -> bf16 / fp16 with gfx950's conversion instructions
// (v_cvt_pk_bf16_f32, v_cvt_f16_f32 / v_cvt_pk_f16_f32): round to nearest,
// ties to even, NaN stays NaN, overflow to infinity.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <int DT_OUT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    if constexpr (DT_OUT == NANOVLLM_GEMM_BF16) {
        return __builtin_bit_cast(uint32_t, bf16x2_t{static_cast<__bf16>(lo), static_cast<__bf16>(hi)});
    } else {
        return __builtin_bit_cast(uint32_t, f16x2_t{static_cast<_Float16>(lo), static_cast<_Float16>(hi)});
    }
}

// Store one fp32 accumulator as the output element type.
template <int DT_OUT>
__device__ __forceinline__ void store_elem(void* c, int64_t idx, float v) {
    if constexpr (DT_OUT == NANOVLLM_GEMM_F32) {
        static_cast<float*>(c)[idx] = v;
    } else if constexpr (DT_OUT == NANOVLLM_GEMM_BF16) {
        static_cast<uint16_t*>(c)[idx] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    } else {
        static_cast<uint16_t*>(c)[idx] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    }
}

// ---------------------------------------------------------------------------
// MFMA wrappers (gfx950).  Operands are 8 packed 16-bit values per lane,
// passed as raw bits.
//
// v_mfma_f32_32x32x16_{bf16,f16}: lane l holds row (l % 32) of the first
// operand and column (l % 32) of the second, at k = 8 * (l / 32) + [0, 8);
// accumulator register v of lane l is D[8*(v/4) + 4*(l/32) + v%4][l % 32].
//
// v_mfma_f32_16x16x32_{bf16,f16}: lane l holds row (l % 16) / column
// (l % 16) at k = 8 * (l / 16) + [0, 8); accumulator v of lane l is
// D[4*(l/16) + v][l % 16].
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ f32x16_t mfma_32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
    if constexpr (DT == NANOVLLM_GEMM_BF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
}

template <int DT>
__device__ __forceinline__ f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
    if constexpr (DT == NANOVLLM_GEMM_BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their no-wait maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const u32x4_t* p) {
    typedef const __attribute__((address_space(3))) u32x4_t* lds_ptr;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)p));
}

// One global_load_lds_dwordx4: lane L copies 16 bytes from its `src` to LDS
// bytes lds + 16 L .. lds + 16 L + 15 (lds must be wave-uniform).
//
// Written as inline assembly rather than __builtin_amdgcn_global_load_lds:
// the compiler models that builtin as pending on both the vector-memory and
// the LDS counters, so while a prefetch is in flight every wait it inserts
// for a fragment ds_read becomes lgkmcnt(0), which drains the reads of the
// next K-step too and serialises LDS reads with the MFMAs.  On gfx950 the
// instruction completes on vmcnt alone (measured: lgkmcnt(0) after it does
// not wait for the data), so the kernels wait on vmcnt explicitly before
// reading what it wrote.  Nothing else in these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}

// dma16 with the non-temporal cache policy (nt), for operands a kernel reads
// exactly once (the weight stream of the decode kernels): their lines do not
// push out of L2 what every workgroup re-reads (A and the prologue inputs).
// Measured on the decode kernel's W copies (bit-identical results, three
// interleaved runs): bf16 6144 x 1024 at M = 4 / 8 / 16 / 32 4.45-4.50 /
// 4.51-4.53 / 4.80-4.82 / 5.69-5.70 -> 4.27-4.32 / 4.32-4.38 / 4.64-4.68 /
// 5.39-5.45 us, the 151936-row LM head at M = 8 / 32 53.8 / 64.9 -> 48.6 /
// 59.5-59.8 us.  The policy gives up the Infinity Cache: with one W
// re-read call after call (resident there, which a model's decode step,
// streaming every layer's weights, never is) M = 32 took 4.68 against
// 3.94 us.  (The same policy on the register loads of gemv_decode moved
// M = 1 by 1%.)
__device__ __forceinline__ void dma16_stream(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// 16-byte global load.
__device__ __forceinline__ u32x4_t load16(const void* p) {
    return *static_cast<const u32x4_t*>(p);
}

// x * sigmoid(x) = x / (1 + e^-x) in fp32 (library exp, IEEE divide; -0 for
// very negative x, where e^-x overflows to infinity).
__device__ __forceinline__ float silu_f32(float x) {
    return x / (1.0f + expf(-x));
}

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) with the hardware base-2 exponential
// and reciprocal (v_exp_f32, v_rcp_f32, each within 1 ulp in fp32): six
// instructions against ~50 for the library exp and IEEE divide, which
// matters because every workgroup of a decode GEMM gates all of A.  Its
// result is rounded to bf16 / fp16 next, where the difference from a
// correctly rounded sigmoid decides the rounding only next to a tie.  Large
// negative x: 2^(+large) = inf, 1 / inf = 0; large positive x: 1 / 1 = 1.
__device__ __forceinline__ float sigmoid_f32(float x) {
    constexpr float kLog2e = 1.44269504088896340736f;
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// fp32 -> one bf16 / fp16 element (round to nearest even; the same
// conversion pack2 applies to pairs).
template <int DT>
__device__ __forceinline__ uint16_t round_half(float x) {
    if constexpr (DT == NANOVLLM_GEMM_BF16) return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
    else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// PRO_GATE on one element: round(a * round(sigmoid(g))).
template <int DT>
__device__ __forceinline__ uint16_t gate1(uint16_t a, uint16_t g) {
    const uint16_t sg = round_half<DT>(sigmoid_f32(half_to_f32<DT>(g)));
    return round_half<DT>(half_to_f32<DT>(a) * half_to_f32<DT>(sg));
}

// PRO_GATE on 8 packed elements: round(a * round(sigmoid(g))), each product
// and sigmoid in fp32, rounding to nearest even in the element type.
template <int DT>
__device__ __forceinline__ u32x4_t gate8(u32x4_t a, u32x4_t g) {
    u32x4_t out;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t sg = pack2<DT>(sigmoid_f32(half_to_f32<DT>(uint16_t(g[q]))),
                                      sigmoid_f32(half_to_f32<DT>(uint16_t(g[q] >> 16))));
        out[q] = pack2<DT>(half_to_f32<DT>(uint16_t(a[q])) * half_to_f32<DT>(uint16_t(sg)),
                           half_to_f32<DT>(uint16_t(a[q] >> 16)) * half_to_f32<DT>(uint16_t(sg >> 16)));
    }
    return out;
}

// PRO_ADD_NORM on 8 packed elements of h, r and the norm weight w: with
// s = h + r in fp32, adds s^2 to ss in element order, returns round(s) (the
// new residual) in res and round(s * (1 + w)) (the GEMM operand).
template <int DT>
__device__ __forceinline__ u32x4_t add_norm8(u32x4_t h, u32x4_t r, u32x4_t w, float& ss, u32x4_t& res) {
    u32x4_t y;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float s0 = half_to_f32<DT>(uint16_t(h[q])) + half_to_f32<DT>(uint16_t(r[q]));
        const float s1 = half_to_f32<DT>(uint16_t(h[q] >> 16)) + half_to_f32<DT>(uint16_t(r[q] >> 16));
        ss = __builtin_fmaf(s0, s0, ss);
        ss = __builtin_fmaf(s1, s1, ss);
        res[q] = pack2<DT>(s0, s1);
        y[q] = pack2<DT>(s0 * (1.0f + half_to_f32<DT>(uint16_t(w[q]))),
                         s1 * (1.0f + half_to_f32<DT>(uint16_t(w[q] >> 16))));
    }
    return y;
}

// rsqrt(ss / k + eps) in fp32 (IEEE divide and square root).
__device__ __forceinline__ float norm_scale(float ss, int64_t k, float eps) {
    return 1.0f / sqrtf(ss / static_cast<float>(k) + eps);
}

// Greedy-argmax key: the fp32 logit mapped to an unsigned integer with the
// same order (sign-magnitude to offset binary) in the high word, and
// 0xFFFFFFFF - column in the low word, so the largest key is the largest
// logit and, among equal logits, the first column (torch.argmax's rule).
// Key 0 is below every real key.
__device__ __forceinline__ uint64_t argmax_key(float v, int64_t col) {
    // -0 ranks equal to +0, and every NaN ranks above every number (as in
    // torch.argmax): both are canonicalised first.
    const uint32_t b = v != v ? 0x7FC00000u : (v == 0.0f ? 0u : __builtin_bit_cast(uint32_t, v));
    const uint32_t ordered = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (uint64_t(ordered) << 32) | uint64_t(0xFFFFFFFFu - uint32_t(col));
}

// Sampled LM head (EPI_ARGMAX with a temperature per row).  Sampler
// (nanovllm/layers/sampler.py:8-21) keeps row i greedy when its temperature
// is <= 1e-10 and otherwise takes argmax_j softmax(v / T)_j / E_j with E_j
// ~ Exp(1) clamped to >= 1e-10.  That is argmax_j (v_j / T - ln E_j), the
// Gumbel-max form, which needs no row-wide softmax: each workgroup ranks its
// own columns by this score and the greedy finalize picks the best key.
// E comes from a counter-based generator so any workgroup can draw the
// noise of any (row, column): u = (24 high bits of word col % 4 of
// Philox4x32-10(counter = (col / 4, row, offset, offset >> 32), key = seed))
// + 1) / 2^24, in (0, 1]; E = max(-ln u, 1e-10).
//
// Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers:
// as easy as 1, 2, 3", SC 2011): ten rounds, each two 32 x 32 -> 64-bit
// products of counter words with the round multipliers, the high halves
// mixed with the other two words and the round key, and the key advanced
// by the Weyl constants between rounds.
__device__ __forceinline__ u32x4_t philox4x32_10(u32x4_t c, uint32_t k0, uint32_t k1) {
    constexpr uint32_t kMul0 = 0xD2511F53u, kMul1 = 0xCD9E8D57u;
    constexpr uint32_t kWeyl0 = 0x9E3779B9u, kWeyl1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = uint64_t(kMul0) * c[0];
        const uint64_t p1 = uint64_t(kMul1) * c[2];
        c = u32x4_t{uint32_t(p1 >> 32) ^ c[1] ^ k0, uint32_t(p1), uint32_t(p0 >> 32) ^ c[3] ^ k1, uint32_t(p0)};
        k0 += kWeyl0;
        k1 += kWeyl1;
    }
    return c;
}

// The value the LM head ranks for an fp32 logit: the logit itself, or its
// round-to-nearest-even image in bf16 / fp16 read back as fp32 (equal
// rounded logits then go to the first column, as torch.argmax does on the
// reference's bf16 logits).  logit_dtype is uniform across the launch.
__device__ __forceinline__ float ranked_logit(float v, const SampleArgs& sa) {
    if (sa.logit_dtype == NANOVLLM_GEMM_BF16) return bf16_to_f32(round_half<NANOVLLM_GEMM_BF16>(v));
    if (sa.logit_dtype == NANOVLLM_GEMM_F16) return f16_to_f32(round_half<NANOVLLM_GEMM_F16>(v));
    return v;
}

// Temperature of a sampled row, 0 for a greedy one (temperature <= 1e-10)
// or when the head is greedy altogether.
__device__ __forceinline__ float sample_temperature(int64_t row, const SampleArgs& sa) {
    if (sa.temperature == nullptr) return 0.0f;
    const float t = sa.temperature[row];
    return t <= 1e-10f ? 0.0f : t;
}

// The four noise words of columns 4 q .. 4 q + 3 of a row.
__device__ __forceinline__ u32x4_t sample_words(int64_t row, int64_t q, const SampleArgs& sa) {
    return philox4x32_10(u32x4_t{uint32_t(q), uint32_t(row), uint32_t(sa.offset), uint32_t(sa.offset >> 32)},
                         uint32_t(sa.seed), uint32_t(sa.seed >> 32));
}

// Score of a sampled column from its logit, the row's temperature and its
// noise word: v / T - ln E (ln from the hardware log2).  gumbel_log2e is
// the part that does not depend on the logit (log2 E), so a kernel can draw
// it before the logit is known; gumbel_apply finishes the score.
__device__ __forceinline__ float gumbel_log2e(uint32_t word) {
    constexpr float kLn2 = 0.693147180559945309f;
    const float u = float((word >> 8) + 1u) * 0x1p-24f;
    const float e = fmaxf(-__builtin_amdgcn_logf(u) * kLn2, 1e-10f);
    return __builtin_amdgcn_logf(e);
}
__device__ __forceinline__ float gumbel_apply(float v, float t, float log2e) {
    constexpr float kLn2 = 0.693147180559945309f;
    return v / t - log2e * kLn2;
}
__device__ __forceinline__ float gumbel_score(float v, float t, uint32_t word) {
    return gumbel_apply(v, t, gumbel_log2e(word));
}

// The score that ranks column col of row row: the ranked logit v (see
// ranked_logit) on a greedy row, v / T - ln E on a sampled one.
__device__ __forceinline__ float sample_score(float v, int64_t row, int64_t col, const SampleArgs& sa) {
    v = ranked_logit(v, sa);
    const float t = sample_temperature(row, sa);
    if (t == 0.0f) return v;
    const u32x4_t x = sample_words(row, col >> 2, sa);
    const int j = int(col & 3);
    return gumbel_score(v, t, j == 0 ? x[0] : j == 1 ? x[1] : j == 2 ? x[2] : x[3]);
}

// Integer minimum.  The device `min` overload set has no exact match for
// 64-bit integers here and resolves to a double-precision one, which costs
// a dozen f64 instructions per call.
__device__ __forceinline__ int64_t min_i64(int64_t x, int64_t y) { return x < y ? x : y; }

// ---------------------------------------------------------------------------
// XCD-aware workgroup order.  Workgroups are handed to the 8 XCDs round
// robin (workgroup w runs on XCD w % 8), and each XCD has its own L2.  The
// remap gives XCD x a contiguous run of logical tile ids, and the grouped
// row-major order below turns such a run into a compact block of tiles
// that share A rows and W rows inside that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_remap(int wg, int total) {
    const int per = total / kNumXcd;
    const int full = per * kNumXcd;
    if (wg >= full) return wg;
    return (wg % kNumXcd) * per + (wg / kNumXcd);
}

// Logical tile id -> (tile_m, tile_n), walking `group_m` tile rows at a
// time so that consecutive ids stay inside a group_m-tall band.
__device__ __forceinline__ void grouped_tile(int t, int tiles_m, int tiles_n, int group_m,
                                             int& tm, int& tn) {
    const int per_group = group_m * tiles_n;
    const int g = t / per_group;
    const int first_m = g * group_m;
    const int rows = min(tiles_m - first_m, group_m);
    const int r = t - g * per_group;
    tm = first_m + r % rows;
    tn = r / rows;
}

// ---------------------------------------------------------------------------
// Launchers (one per kernel family).  Each returns NANOVLLM_GEMM_OK or a
// negative code; the caller has already validated the problem and checked
// that the kernel supports it.
// ---------------------------------------------------------------------------
int launch_fp32_naive(const Problem& p, hipStream_t s);
int launch_fp32_tiled(const Problem& p, hipStream_t s);
int launch_mfma_direct(const Problem& p, hipStream_t s);
int launch_mfma_staged(const Problem& p, hipStream_t s);
int launch_splitk_decode(const Problem& p, hipStream_t s);
int launch_gemv_decode(const Problem& p, hipStream_t s);

// Reduces `blocks` partial keys per row ([m, blocks], from an EPI_ARGMAX
// launch) to the greedy token of each row (int64) and, if `logits` is not
// null, its logit.
// Standalone prologues (gemm_prologue.hip): the GEMM operand written to a
// buffer, for the problems the fused decode kernel does not take.
int launch_gate_prologue(const void* a, int64_t lda, const void* g, int64_t ldg, int64_t group,
                         int64_t group_stride, void* out, int64_t ldo, int64_t m, int64_t k, int dtype,
                         hipStream_t s);
int launch_add_norm_prologue(const void* h, int64_t ldh, const void* r, int64_t ldr, const void* w, float eps,
                             void* y, int64_t ldy, void* res, int64_t ldres, float* scale, int64_t m, int64_t k,
                             int dtype, hipStream_t s);
int launch_argmax_finalize(const uint64_t* keys, int64_t blocks, int64_t m, int64_t* tokens, float* logits,
                           hipStream_t s);

// Bytes of the device scratch array behind nanovllm_gemm_argmax_noalloc, and
// its address on the device of `stream` (resolved once per device).
constexpr int64_t kArgmaxScratchBytes = int64_t(8) << 20;
int argmax_scratch(hipStream_t stream, void** ptr);

// Records a message for nanovllm_gemm_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

// Converts a hipError_t after a launch into a return code.
int check_launch(const char* kernel);

}  // namespace nvg
