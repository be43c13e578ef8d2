// C ABI of libnanovllm_gemm.so: argument validation, the shape-selection
// table, dispatch to the kernel launchers, and thread-local error text.
// Declarations and their reference counterparts: include/nanovllm_gemm.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "gemm_common.hpp"

namespace nvg {

namespace {
thread_local std::string g_last_error;

bool dtype_pair_ok(int din, int dout) {
    switch (din) {
        case NANOVLLM_GEMM_F32: return dout == NANOVLLM_GEMM_F32;
        case NANOVLLM_GEMM_F16: return dout == NANOVLLM_GEMM_F16 || dout == NANOVLLM_GEMM_F32;
        case NANOVLLM_GEMM_BF16: return dout == NANOVLLM_GEMM_BF16 || dout == NANOVLLM_GEMM_F32;
        default: return false;
    }
}

bool is_half(int dt) { return dt == NANOVLLM_GEMM_F16 || dt == NANOVLLM_GEMM_BF16; }

// Checks sizes, strides and enums; records the reason on failure.
int validate(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int b_layout, int din,
             int dout) {
    if (b_layout != NANOVLLM_GEMM_B_NK && b_layout != NANOVLLM_GEMM_B_KN)
        return set_error(NANOVLLM_GEMM_EINVAL, "b_layout must be NANOVLLM_GEMM_B_NK (0) or NANOVLLM_GEMM_B_KN (1), got %d",
                         b_layout);
    if (din < NANOVLLM_GEMM_F32 || din > NANOVLLM_GEMM_BF16 || dout < NANOVLLM_GEMM_F32 || dout > NANOVLLM_GEMM_BF16)
        return set_error(NANOVLLM_GEMM_EINVAL, "unknown dtype code (in %d, out %d)", din, dout);
    if (!dtype_pair_ok(din, dout))
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "unsupported dtype pair (in %d, out %d): supported are f32->f32, f16->{f16,f32}, "
                         "bf16->{bf16,f32}",
                         din, dout);
    if (m < 0 || n < 0) return set_error(NANOVLLM_GEMM_EINVAL, "m and n must be non-negative (m=%lld, n=%lld)",
                                         (long long)m, (long long)n);
    if (k < 1) return set_error(NANOVLLM_GEMM_EINVAL, "k must be positive (k=%lld)", (long long)k);
    if (lda < k) return set_error(NANOVLLM_GEMM_EINVAL, "lda (%lld) must be >= k (%lld)", (long long)lda, (long long)k);
    const int64_t ldb_min = b_layout == NANOVLLM_GEMM_B_NK ? k : n;
    if (ldb < ldb_min || ldb < 1)
        return set_error(NANOVLLM_GEMM_EINVAL, "ldb (%lld) must be >= %s (%lld)", (long long)ldb,
                         b_layout == NANOVLLM_GEMM_B_NK ? "k" : "n", (long long)ldb_min);
    if (ldc < n || ldc < 1)
        return set_error(NANOVLLM_GEMM_EINVAL, "ldc (%lld) must be >= n (%lld)", (long long)ldc, (long long)n);
    return NANOVLLM_GEMM_OK;
}

// Half-precision problems whose rows can be read as aligned 16-byte chunks.
bool vector_ok(int64_t k, int64_t lda, int64_t ldb, int b_layout, int aligned16) {
    return aligned16 && k % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && b_layout == NANOVLLM_GEMM_B_NK;
}

// B[K,N] problems mfma_staged reads in 16-byte chunks: rows of A as above,
// and rows of B in whole 8-column chunks (N a multiple of 8).
bool kn_vector_ok(int64_t n, int64_t k, int64_t lda, int64_t ldb, int b_layout, int aligned16) {
    return aligned16 && k % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && n % 8 == 0 && b_layout == NANOVLLM_GEMM_B_KN;
}

// M at or below this is streamed by splitk_decode: the problem is bound by
// reading W once (arithmetic intensity ~M flop/byte, far under the
// ~312 flop/byte bf16 ridge of MI355X).
constexpr int64_t kDecodeMaxM = 32;

// The plain GEMM also runs on splitk_decode up to M = 64 when W has fewer
// than 65536 rows.  The table picks it there for narrow problems, where
// mfma_staged's 64 x 64 tiles leave most CUs idle (bf16, M = 64: N = 1024,
// K = 3584 6.5 against 15.5 us; N = 4096, K = 4096 10.0 against 19.0 us;
// N = 8224, K = 1024 5.7 against 6.2 us), and not from 16384 rows or, above
// 4096 rows, beyond K = 1024 (N = 12288, K = 2048: 14.3 against 11.6 us).
constexpr int64_t kSplitkPlainMaxM = 64;
constexpr int64_t kSplitkPlainMaxRows = 65535;
constexpr int64_t kSplitkPlainNarrowN = 4096;
constexpr int64_t kSplitkPlainShortKMaxN = 10240;
constexpr int64_t kSplitkPlainShortK = 1024;

constexpr int64_t kSplitkSiluMaxRows = 16384;

bool splitk_plain_ok(int64_t m, int64_t n) {
    return m <= kDecodeMaxM || (m <= kSplitkPlainMaxM && n <= kSplitkPlainMaxRows);
}

bool supports(int kernel_id, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int b_layout, int din,
              int aligned16) {
    switch (kernel_id) {
        case NANOVLLM_GEMM_KERNEL_FP32_NAIVE:
        case NANOVLLM_GEMM_KERNEL_FP32_TILED: return din == NANOVLLM_GEMM_F32;
        case NANOVLLM_GEMM_KERNEL_MFMA_DIRECT: return is_half(din);
        case NANOVLLM_GEMM_KERNEL_MFMA_STAGED:
            return is_half(din) &&
                   (vector_ok(k, lda, ldb, b_layout, aligned16) || kn_vector_ok(n, k, lda, ldb, b_layout, aligned16));
        case NANOVLLM_GEMM_KERNEL_SPLITK_DECODE:
            return is_half(din) && ((vector_ok(k, lda, ldb, b_layout, aligned16) && splitk_plain_ok(m, n)) ||
                                    (kn_vector_ok(n, k, lda, ldb, b_layout, aligned16) && m <= kSplitkPlainMaxM));
        case NANOVLLM_GEMM_KERNEL_GEMV_DECODE:
            return is_half(din) && vector_ok(k, lda, ldb, b_layout, aligned16) && m == 1;
        default: return false;
    }
}

// M = 1 with a W of at most this many bytes goes to gemv_decode: its many
// small workgroups win when the stream is short (12.6 MB: 4.5 vs 5.0 us on
// MI355X), while for long streams (the 311 MB LM head) splitk_decode's
// longer per-lane runs are faster (53 vs 64 us).
constexpr int64_t kGemvMaxWBytes = int64_t(64) << 20;

// The shape-selection table (replaces supports_wmma + choose_path,
// cuda_kernels/gemm/src/gemm_bench.cu:252-273).  Every valid problem maps
// to a kernel of this library; there is no vendor fallback.
int select(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int b_layout, int din, int aligned16) {
    if (din == NANOVLLM_GEMM_F32) return NANOVLLM_GEMM_KERNEL_FP32_TILED;
    if (vector_ok(k, lda, ldb, b_layout, aligned16)) {
        if (m == 1 && n * k * 2 <= kGemvMaxWBytes) return NANOVLLM_GEMM_KERNEL_GEMV_DECODE;
        if (m <= kDecodeMaxM) return NANOVLLM_GEMM_KERNEL_SPLITK_DECODE;
        if (m <= kSplitkPlainMaxM &&
            (n <= kSplitkPlainNarrowN || (n <= kSplitkPlainShortKMaxN && k <= kSplitkPlainShortK)))
            return NANOVLLM_GEMM_KERNEL_SPLITK_DECODE;
        return NANOVLLM_GEMM_KERNEL_MFMA_STAGED;
    }
    // B[K,N] (the reference bench's layout): splitk_decode up to M = 32 and
    // up to M = 64 on at most 4096 columns, the staged kernel above.  On the
    // reference's shape matrix (bf16, fp32 out) splitk_decode took M = 1 / 16
    // from 6.2-9.9 us (staged) to 3.7-4.6 us, and 64 x 1024 x 2048 / 3584
    // from 10.0 / 15.8 to 8.1 / 10.8 us; at 64 x 6144 / 7168 (96 / 112
    // workgroups of 64 columns) it ran 6.8 / 7.0 against 6.6 / 6.7 us.
    if (kn_vector_ok(n, k, lda, ldb, b_layout, aligned16)) {
        if (m <= kDecodeMaxM || (m <= kSplitkPlainMaxM && n <= kSplitkPlainNarrowN))
            return NANOVLLM_GEMM_KERNEL_SPLITK_DECODE;
        return NANOVLLM_GEMM_KERNEL_MFMA_STAGED;
    }
    return NANOVLLM_GEMM_KERNEL_MFMA_DIRECT;
}

int run(int kernel_id, const Problem& p, hipStream_t s) {
    switch (kernel_id) {
        case NANOVLLM_GEMM_KERNEL_FP32_NAIVE: return launch_fp32_naive(p, s);
        case NANOVLLM_GEMM_KERNEL_FP32_TILED: return launch_fp32_tiled(p, s);
        case NANOVLLM_GEMM_KERNEL_MFMA_DIRECT: return launch_mfma_direct(p, s);
        case NANOVLLM_GEMM_KERNEL_MFMA_STAGED: return launch_mfma_staged(p, s);
        case NANOVLLM_GEMM_KERNEL_SPLITK_DECODE: return launch_splitk_decode(p, s);
        case NANOVLLM_GEMM_KERNEL_GEMV_DECODE: return launch_gemv_decode(p, s);
        default: return set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel_id);
    }
}

int aligned16_of(const void* a, const void* b) {
    return (reinterpret_cast<uintptr_t>(a) % 16 == 0) && (reinterpret_cast<uintptr_t>(b) % 16 == 0);
}

int gemm_entry(int forced_kernel, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
               int64_t lda, int64_t ldb, int64_t ldc, int b_layout, int din, int dout, void* stream) {
    g_last_error.clear();
    int rc = validate(m, n, k, lda, ldb, ldc, b_layout, din, dout);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m == 0 || n == 0) return NANOVLLM_GEMM_OK;
    if (a == nullptr || b == nullptr || c == nullptr)
        return set_error(NANOVLLM_GEMM_EINVAL, "a, b and c must be non-null device pointers");
    const int al = aligned16_of(a, b);
    int kernel = forced_kernel;
    if (kernel < 0) {
        kernel = select(m, n, k, lda, ldb, b_layout, din, al);
    } else if (kernel >= NANOVLLM_GEMM_KERNEL_COUNT) {
        return set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel);
    } else if (!supports(kernel, m, n, k, lda, ldb, b_layout, din, al)) {
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "kernel %s cannot run this problem (m=%lld n=%lld k=%lld)",
                         nanovllm_gemm_kernel_name(kernel), (long long)m, (long long)n, (long long)k);
    }
    const Problem p{a, b, c, m, n, k, lda, ldb, ldc, b_layout, din, dout};
    return run(kernel, p, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Fused gate/up projection + SiLU-and-mul: c[M, n] from W = [W_gate; W_up]
// of 2n rows in the W[N,K] layout.  Runs on the vector-path kernels only.
// ---------------------------------------------------------------------------
int validate_silu_mul(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw, int64_t ldc, int din, int dout) {
    if (din < NANOVLLM_GEMM_F32 || din > NANOVLLM_GEMM_BF16 || dout < NANOVLLM_GEMM_F32 || dout > NANOVLLM_GEMM_BF16)
        return set_error(NANOVLLM_GEMM_EINVAL, "unknown dtype code (in %d, out %d)", din, dout);
    if (!is_half(din) || !dtype_pair_ok(din, dout))
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "unsupported dtype pair for silu_mul (in %d, out %d): supported are f16->{f16,f32}, "
                         "bf16->{bf16,f32}",
                         din, dout);
    if (m < 0 || n < 0) return set_error(NANOVLLM_GEMM_EINVAL, "m and n must be non-negative (m=%lld, n=%lld)",
                                         (long long)m, (long long)n);
    if (k < 1) return set_error(NANOVLLM_GEMM_EINVAL, "k must be positive (k=%lld)", (long long)k);
    if (lda < k) return set_error(NANOVLLM_GEMM_EINVAL, "lda (%lld) must be >= k (%lld)", (long long)lda, (long long)k);
    if (ldw < k) return set_error(NANOVLLM_GEMM_EINVAL, "ldw (%lld) must be >= k (%lld)", (long long)ldw, (long long)k);
    if (ldc < n || ldc < 1)
        return set_error(NANOVLLM_GEMM_EINVAL, "ldc (%lld) must be >= n (%lld)", (long long)ldc, (long long)n);
    return NANOVLLM_GEMM_OK;
}

bool supports_silu_mul(int kernel_id, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw, int aligned16) {
    if (!vector_ok(k, lda, ldw, NANOVLLM_GEMM_B_NK, aligned16)) return false;
    switch (kernel_id) {
        case NANOVLLM_GEMM_KERNEL_MFMA_STAGED: return true;
        case NANOVLLM_GEMM_KERNEL_SPLITK_DECODE: return splitk_plain_ok(m, 2 * n);
        case NANOVLLM_GEMM_KERNEL_GEMV_DECODE: return m == 1;
        default: return false;
    }
}

// Same regimes as select(): the fused epilogue does not change what bounds
// each shape.
int select_silu_mul(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw, int aligned16) {
    if (!vector_ok(k, lda, ldw, NANOVLLM_GEMM_B_NK, aligned16))
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "silu_mul needs 16-byte aligned a and w with k, lda and ldw multiples of 8 "
                         "(k=%lld lda=%lld ldw=%lld)",
                         (long long)k, (long long)lda, (long long)ldw);
    // M = 1 included: on the Qwen3.5-0.8B gate_up_proj (2 x 3584 rows, K =
    // 1024) splitk_decode's whole-line copies take 4.9 us against 5.2 us for
    // gemv_decode streaming the gate and up rows.
    if (m <= kDecodeMaxM) return NANOVLLM_GEMM_KERNEL_SPLITK_DECODE;
    // 33 <= M <= 64: mfma_staged's SiLU grid is one row of 64 x 128 tiles;
    // splitk_decode spreads the gate/up pairs over 2n / 32 workgroups (bf16,
    // K = 1024, M = 64: n = 3584 4.7 against 9.2 us, n = 8192 9.7 against
    // 11.9 us; K = 2048, n = 3584: 8.1 against 15.1 us).
    if (m <= kSplitkPlainMaxM && 2 * n <= kSplitkSiluMaxRows) return NANOVLLM_GEMM_KERNEL_SPLITK_DECODE;
    return NANOVLLM_GEMM_KERNEL_MFMA_STAGED;
}

int silu_mul_entry(int forced_kernel, const void* a, const void* w, void* c, int64_t m, int64_t n, int64_t k,
                   int64_t lda, int64_t ldw, int64_t ldc, int din, int dout, void* stream) {
    g_last_error.clear();
    int rc = validate_silu_mul(m, n, k, lda, ldw, ldc, din, dout);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m == 0 || n == 0) return NANOVLLM_GEMM_OK;
    if (a == nullptr || w == nullptr || c == nullptr)
        return set_error(NANOVLLM_GEMM_EINVAL, "a, w and c must be non-null device pointers");
    const int al = aligned16_of(a, w);
    int kernel = forced_kernel;
    if (kernel < 0) {
        kernel = select_silu_mul(m, n, k, lda, ldw, al);
        if (kernel < 0) return kernel;
    } else if (!supports_silu_mul(kernel, m, n, k, lda, ldw, al)) {
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "kernel %s cannot run silu_mul for this problem (m=%lld n=%lld k=%lld)",
                         nanovllm_gemm_kernel_name(kernel), (long long)m, (long long)n, (long long)k);
    }
    Problem p{a, w, c, m, n, k, lda, ldw, ldc, NANOVLLM_GEMM_B_NK, din, dout};
    p.epi = EPI_SILU_MUL;
    return run(kernel, p, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Greedy LM head: token = argmax_j (a W^T)[i, j] per row, without writing the
// logits.  Partial keys per workgroup go to a caller-provided workspace.
// ---------------------------------------------------------------------------
int validate_argmax(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw, int din) {
    if (din != NANOVLLM_GEMM_F16 && din != NANOVLLM_GEMM_BF16)
        return set_error(din >= NANOVLLM_GEMM_F32 && din <= NANOVLLM_GEMM_BF16 ? NANOVLLM_GEMM_EUNSUPPORTED
                                                                               : NANOVLLM_GEMM_EINVAL,
                         "argmax takes float16 or bfloat16 inputs (dtype code %d)", din);
    if (m < 0) return set_error(NANOVLLM_GEMM_EINVAL, "m must be non-negative (m=%lld)", (long long)m);
    if (n < 1 || n > INT64_C(0xFFFFFFFF))
        return set_error(NANOVLLM_GEMM_EINVAL, "n must be in [1, 2^32) (n=%lld)", (long long)n);
    if (k < 1) return set_error(NANOVLLM_GEMM_EINVAL, "k must be positive (k=%lld)", (long long)k);
    if (lda < k) return set_error(NANOVLLM_GEMM_EINVAL, "lda (%lld) must be >= k (%lld)", (long long)lda, (long long)k);
    if (ldw < k) return set_error(NANOVLLM_GEMM_EINVAL, "ldw (%lld) must be >= k (%lld)", (long long)ldw, (long long)k);
    return NANOVLLM_GEMM_OK;
}

bool supports_argmax(int kernel_id, int64_t m, int64_t k, int64_t lda, int64_t ldw, int aligned16) {
    if (!vector_ok(k, lda, ldw, NANOVLLM_GEMM_B_NK, aligned16)) return false;
    if (kernel_id == NANOVLLM_GEMM_KERNEL_SPLITK_DECODE) return m <= kDecodeMaxM;
    return kernel_id == NANOVLLM_GEMM_KERNEL_MFMA_STAGED;
}

int select_argmax(int64_t m, int64_t k, int64_t lda, int64_t ldw, int aligned16) {
    if (!vector_ok(k, lda, ldw, NANOVLLM_GEMM_B_NK, aligned16))
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "argmax needs 16-byte aligned a and w with k, lda and ldw multiples of 8 "
                         "(k=%lld lda=%lld ldw=%lld)",
                         (long long)k, (long long)lda, (long long)ldw);
    return m <= kDecodeMaxM ? NANOVLLM_GEMM_KERNEL_SPLITK_DECODE : NANOVLLM_GEMM_KERNEL_MFMA_STAGED;
}

// Bytes of partial keys any kernel that can run the problem writes: one
// 8-byte key per row of A per workgroup along N (split-K workgroups cover at
// least 16 columns, staged tiles 128).
int64_t argmax_workspace_bytes(int64_t m, int64_t n) {
    const int64_t cols_per_block = m <= kDecodeMaxM ? 16 : 128;
    return ((n + cols_per_block - 1) / cols_per_block) * m * int64_t(sizeof(uint64_t));
}

// The LM head ranks the fp32 accumulator (logit_dt f32) or its rounding to
// the input type (logit_dt == din: the logits F.linear returns in the model
// dtype, nanovllm/layers/embed_head.py:61).
int validate_logit_dtype(int din, int logit_dt) {
    if (logit_dt != NANOVLLM_GEMM_F32 && logit_dt != din)
        return set_error(NANOVLLM_GEMM_EINVAL,
                         "logit_dtype must be NANOVLLM_GEMM_F32 (0) or the input dtype (%d), got %d", din, logit_dt);
    return NANOVLLM_GEMM_OK;
}

// `sample`: nullptr for the greedy head; the sampled head passes its
// per-row temperatures (device memory, required) and noise seed / offset.
int argmax_entry(int forced_kernel, const void* a, const void* w, int64_t* tokens, float* logits, int64_t m,
                 int64_t n, int64_t k, int64_t lda, int64_t ldw, int din, int logit_dt, void* workspace,
                 int64_t workspace_bytes, void* stream, const SampleArgs* sample = nullptr) {
    g_last_error.clear();
    int rc = validate_argmax(m, n, k, lda, ldw, din);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    rc = validate_logit_dtype(din, logit_dt);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m == 0) return NANOVLLM_GEMM_OK;
    if (a == nullptr || w == nullptr || tokens == nullptr || workspace == nullptr)
        return set_error(NANOVLLM_GEMM_EINVAL, "a, w, tokens and workspace must be non-null device pointers");
    if (sample != nullptr && sample->temperature == nullptr)
        return set_error(NANOVLLM_GEMM_EINVAL, "temperatures must be a non-null device pointer to m floats");
    if (sample != nullptr && reinterpret_cast<uintptr_t>(sample->temperature) % 4 != 0)
        return set_error(NANOVLLM_GEMM_EINVAL, "temperatures must be 4-byte aligned");
    if (reinterpret_cast<uintptr_t>(workspace) % 8 != 0)
        return set_error(NANOVLLM_GEMM_EINVAL, "workspace must be 8-byte aligned");
    const int64_t need = argmax_workspace_bytes(m, n);
    if (workspace_bytes < need)
        return set_error(NANOVLLM_GEMM_EINVAL, "workspace of %lld bytes is too small: this problem needs %lld",
                         (long long)workspace_bytes, (long long)need);
    const int al = aligned16_of(a, w);
    int kernel = forced_kernel;
    if (kernel < 0) {
        kernel = select_argmax(m, k, lda, ldw, al);
        if (kernel < 0) return kernel;
    } else if (!supports_argmax(kernel, m, k, lda, ldw, al)) {
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "kernel %s cannot run argmax for this problem (m=%lld n=%lld k=%lld)",
                         nanovllm_gemm_kernel_name(kernel), (long long)m, (long long)n, (long long)k);
    }
    int64_t blocks = 0;
    Problem p{a, w, nullptr, m, n, k, lda, ldw, n, NANOVLLM_GEMM_B_NK, din, NANOVLLM_GEMM_F32};
    p.epi = EPI_ARGMAX;
    p.keys = static_cast<uint64_t*>(workspace);
    p.key_blocks = &blocks;
    if (sample != nullptr) p.sample = *sample;
    p.sample.logit_dtype = logit_dt;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    rc = run(kernel, p, s);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    return launch_argmax_finalize(p.keys, blocks, m, tokens, logits, s);
}

// ---------------------------------------------------------------------------
// GEMMs with a prologue on A: the gated-attention output gate before o_proj
// and the residual add + zero-centred RMSNorm before a projection.  For
// M <= 32 the prologue runs inside splitk_decode (one launch); otherwise a
// prologue kernel writes the operand to the workspace and the GEMM reads it.
// ---------------------------------------------------------------------------
bool aligned16_ptr(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int64_t round_up_256(int64_t x) { return (x + 255) / 256 * 256; }

int validate_prologue_dtypes(int din, int dout, const char* what) {
    if (din != NANOVLLM_GEMM_F16 && din != NANOVLLM_GEMM_BF16)
        return set_error(din >= NANOVLLM_GEMM_F32 && din <= NANOVLLM_GEMM_BF16 ? NANOVLLM_GEMM_EUNSUPPORTED
                                                                               : NANOVLLM_GEMM_EINVAL,
                         "%s takes float16 or bfloat16 inputs (dtype code %d)", what, din);
    if (dout != din && dout != NANOVLLM_GEMM_F32)
        return set_error(dout >= NANOVLLM_GEMM_F32 && dout <= NANOVLLM_GEMM_BF16 ? NANOVLLM_GEMM_EUNSUPPORTED
                                                                                 : NANOVLLM_GEMM_EINVAL,
                         "%s writes the input dtype or float32 (dtype codes in %d, out %d)", what, din, dout);
    return NANOVLLM_GEMM_OK;
}

// Sizes and strides of the gated GEMM; the vector path's alignment is
// checked separately (gated_vector_ok).
int validate_gated(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldg, int64_t group, int64_t group_stride,
                   int64_t ldw, int64_t ldc, int din, int dout) {
    int rc = validate_prologue_dtypes(din, dout, "gemm_gated");
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m < 0 || n < 0) return set_error(NANOVLLM_GEMM_EINVAL, "m and n must be non-negative (m=%lld, n=%lld)",
                                         (long long)m, (long long)n);
    if (k < 1) return set_error(NANOVLLM_GEMM_EINVAL, "k must be positive (k=%lld)", (long long)k);
    if (group < 1 || k % group != 0)
        return set_error(NANOVLLM_GEMM_EINVAL, "group (%lld) must divide k (%lld)", (long long)group, (long long)k);
    if (group_stride < group)
        return set_error(NANOVLLM_GEMM_EINVAL, "group_stride (%lld) must be >= group (%lld)", (long long)group_stride,
                         (long long)group);
    const int64_t gate_row = (k / group - 1) * group_stride + group;   // elements one gate row spans
    if (ldg < gate_row)
        return set_error(NANOVLLM_GEMM_EINVAL, "ldg (%lld) must be >= %lld, the span of one gate row",
                         (long long)ldg, (long long)gate_row);
    if (lda < k) return set_error(NANOVLLM_GEMM_EINVAL, "lda (%lld) must be >= k (%lld)", (long long)lda, (long long)k);
    if (ldw < k) return set_error(NANOVLLM_GEMM_EINVAL, "ldw (%lld) must be >= k (%lld)", (long long)ldw, (long long)k);
    if (ldc < n || ldc < 1)
        return set_error(NANOVLLM_GEMM_EINVAL, "ldc (%lld) must be >= n (%lld)", (long long)ldc, (long long)n);
    return NANOVLLM_GEMM_OK;
}

bool gated_vector_ok(int64_t k, int64_t lda, int64_t ldg, int64_t group, int64_t group_stride, int64_t ldw,
                     int aligned16) {
    return vector_ok(k, lda, ldw, NANOVLLM_GEMM_B_NK, aligned16) && ldg % 8 == 0 && group % 8 == 0 &&
           group_stride % 8 == 0;
}

// The fused gate runs inside splitk_decode up to this M.  Every workgroup
// gates all of A, so the sigmoids grow with M times the workgroup count; on
// the Qwen3.5 o_proj (N = 1024, K = 2048) fused / gate kernel + GEMM measured
// 4.7 / 5.4 us at M = 1, 6.1 / 6.6 us at M = 8, 9.9 / 7.0 us at M = 16.
constexpr int64_t kGateFusedMaxM = 8;

// The fused path copies whole 64-element lines of the gate, so a line must
// not straddle two gate groups.
bool gated_fused(int64_t m, int64_t group) { return m <= kGateFusedMaxM && group % 64 == 0; }

// Enough for any kernel that can run the problem (the fused gate uses none).
int64_t gated_workspace_bytes(int64_t m, int64_t k) { return round_up_256(m * k * 2); }

int gated_entry(int forced_kernel, const void* a, const void* gate, const void* w, void* c, int64_t m, int64_t n,
                int64_t k, int64_t lda, int64_t ldg, int64_t group, int64_t group_stride, int64_t ldw, int64_t ldc,
                int din, int dout, void* workspace, int64_t workspace_bytes, void* stream) {
    g_last_error.clear();
    int rc = validate_gated(m, n, k, lda, ldg, group, group_stride, ldw, ldc, din, dout);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m == 0 || n == 0) return NANOVLLM_GEMM_OK;
    if (a == nullptr || gate == nullptr || w == nullptr || c == nullptr)
        return set_error(NANOVLLM_GEMM_EINVAL, "a, gate, w and c must be non-null device pointers");
    const int al = aligned16_ptr(a) && aligned16_ptr(gate) && aligned16_ptr(w);
    if (!gated_vector_ok(k, lda, ldg, group, group_stride, ldw, al))
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "gemm_gated needs 16-byte aligned a, gate and w with k, lda, ldg, group, group_stride "
                         "and ldw multiples of 8");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool fused = forced_kernel < 0 ? gated_fused(m, group) : forced_kernel == NANOVLLM_GEMM_KERNEL_SPLITK_DECODE;
    if (fused) {
        if (!(m <= kDecodeMaxM && group % 64 == 0))
            return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                             "the fused gate runs in splitk_decode for m <= 32 and group a multiple of 64 "
                             "(m=%lld group=%lld)", (long long)m, (long long)group);
        Problem p{a, w, c, m, n, k, lda, ldw, ldc, NANOVLLM_GEMM_B_NK, din, dout};
        p.pro = PRO_GATE;
        p.a2 = gate;
        p.lda2 = ldg;
        p.group = group;
        p.group_stride = group_stride;
        return launch_splitk_decode(p, s);
    }
    // The gated operand goes to the workspace (leading dimension k), then the
    // GEMM the table (or the caller) picks for it.
    const int64_t need = round_up_256(m * k * 2);
    if (workspace == nullptr || workspace_bytes < need || !aligned16_ptr(workspace))
        return set_error(NANOVLLM_GEMM_EINVAL,
                         "this problem needs a 16-byte aligned workspace of %lld bytes (got %lld)", (long long)need,
                         (long long)workspace_bytes);
    int kernel = forced_kernel < 0 ? select(m, n, k, k, ldw, NANOVLLM_GEMM_B_NK, din, 1) : forced_kernel;
    if (forced_kernel >= NANOVLLM_GEMM_KERNEL_COUNT || !supports(kernel, m, n, k, k, ldw, NANOVLLM_GEMM_B_NK, din, 1))
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "kernel %s cannot run the gated GEMM (m=%lld n=%lld k=%lld)",
                         nanovllm_gemm_kernel_name(kernel), (long long)m, (long long)n, (long long)k);
    rc = launch_gate_prologue(a, lda, gate, ldg, group, group_stride, workspace, k, m, k, din, s);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    const Problem p{workspace, w, c, m, n, k, k, ldw, ldc, NANOVLLM_GEMM_B_NK, din, dout};
    return run(kernel, p, s);
}

// The fused norm rounds s (1 + w) to the input type and applies the row scale
// rsqrt(mean s^2 + eps) after the GEMM, where the reference rounds the O(1)
// product s rsqrt(...) (1 + w).  bf16 has fp32's exponent range, so both
// orders stay finite and normal on any fp32 s; fp16 would overflow where
// |s (1 + w)| > 65504 and go subnormal on rows of small s, where the
// reference stays finite and normal.  fp16 is therefore refused.
int validate_add_norm_dtypes(int din, int dout) {
    const int rc = validate_prologue_dtypes(din, dout, "gemm_add_rmsnorm");
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (din != NANOVLLM_GEMM_BF16)
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "gemm_add_rmsnorm takes bfloat16 inputs only: it rounds s*(1+w) before the row scale, "
                         "which overflows or underflows float16 on rows the reference normalises first");
    return NANOVLLM_GEMM_OK;
}

int validate_add_norm(int64_t m, int64_t n, int64_t k, int64_t ldh, int64_t ldr, int64_t ldw, int64_t ldc,
                      int64_t ldres, float eps, int din, int dout) {
    int rc = validate_add_norm_dtypes(din, dout);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m < 0) return set_error(NANOVLLM_GEMM_EINVAL, "m must be non-negative (m=%lld)", (long long)m);
    if (n < 1) return set_error(NANOVLLM_GEMM_EINVAL, "n must be positive (n=%lld)", (long long)n);
    if (k < 1) return set_error(NANOVLLM_GEMM_EINVAL, "k must be positive (k=%lld)", (long long)k);
    if (!(eps >= 0.0f) || eps > 1.0f) return set_error(NANOVLLM_GEMM_EINVAL, "eps must be in [0, 1]");
    if (ldh < k || ldr < k || ldres < k)
        return set_error(NANOVLLM_GEMM_EINVAL, "ldh, ldr and ldres (%lld, %lld, %lld) must be >= k (%lld)",
                         (long long)ldh, (long long)ldr, (long long)ldres, (long long)k);
    if (ldw < k) return set_error(NANOVLLM_GEMM_EINVAL, "ldw (%lld) must be >= k (%lld)", (long long)ldw, (long long)k);
    if (ldc < n || ldc < 1)
        return set_error(NANOVLLM_GEMM_EINVAL, "ldc (%lld) must be >= n (%lld)", (long long)ldc, (long long)n);
    return NANOVLLM_GEMM_OK;
}

// Operand y at the start of the workspace (leading dimension k), then the
// fp32 row scales; enough for either kernel (the fused norm uses none).
int64_t add_norm_workspace_bytes(int64_t m, int64_t k) { return round_up_256(m * k * 2) + round_up_256(m * 4); }

int add_norm_entry(int forced_kernel, const void* h, const void* r, const void* norm_w, float eps, const void* w,
                   void* c, void* res_out, int64_t m, int64_t n, int64_t k, int64_t ldh, int64_t ldr, int64_t ldw,
                   int64_t ldc, int64_t ldres, int silu_mul, int din, int dout, void* workspace,
                   int64_t workspace_bytes, void* stream) {
    g_last_error.clear();
    int rc = validate_add_norm(m, n, k, ldh, ldr, ldw, ldc, ldres, eps, din, dout);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m == 0) return NANOVLLM_GEMM_OK;
    if (h == nullptr || r == nullptr || norm_w == nullptr || w == nullptr || res_out == nullptr || c == nullptr)
        return set_error(NANOVLLM_GEMM_EINVAL, "h, residual, norm_weight, w, c and residual_out must be non-null");
    const bool al = aligned16_ptr(h) && aligned16_ptr(r) && aligned16_ptr(norm_w) && aligned16_ptr(w) &&
                    aligned16_ptr(res_out);
    if (!(al && k % 8 == 0 && ldh % 8 == 0 && ldr % 8 == 0 && ldres % 8 == 0 && ldw % 8 == 0))
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                         "gemm_add_rmsnorm needs 16-byte aligned h, residual, norm_weight, w and residual_out "
                         "with k, ldh, ldr, ldres and ldw multiples of 8");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool fused = forced_kernel < 0 ? m <= kDecodeMaxM : forced_kernel == NANOVLLM_GEMM_KERNEL_SPLITK_DECODE;
    if (fused) {
        if (m > kDecodeMaxM)
            return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "the fused norm runs in splitk_decode for m <= 32 (m=%lld)",
                             (long long)m);
        Problem p{h, w, c, m, n, k, ldh, ldw, ldc, NANOVLLM_GEMM_B_NK, din, dout};
        p.epi = silu_mul ? EPI_SILU_MUL : EPI_NONE;
        p.pro = PRO_ADD_NORM;
        p.a2 = r;
        p.lda2 = ldr;
        p.norm_w = norm_w;
        p.eps = eps;
        p.res_out = res_out;
        p.ldres = ldres;
        return launch_splitk_decode(p, s);
    }
    if (forced_kernel >= 0 && forced_kernel != NANOVLLM_GEMM_KERNEL_MFMA_STAGED)
        return set_error(NANOVLLM_GEMM_EUNSUPPORTED, "gemm_add_rmsnorm runs on splitk_decode or mfma_staged, not %s",
                         nanovllm_gemm_kernel_name(forced_kernel));
    const int64_t y_bytes = round_up_256(m * k * 2);
    const int64_t need = y_bytes + round_up_256(m * 4);
    if (workspace == nullptr || workspace_bytes < need || !aligned16_ptr(workspace))
        return set_error(NANOVLLM_GEMM_EINVAL,
                         "this problem needs a 16-byte aligned workspace of %lld bytes (got %lld)", (long long)need,
                         (long long)workspace_bytes);
    float* scale = reinterpret_cast<float*>(static_cast<char*>(workspace) + y_bytes);
    rc = launch_add_norm_prologue(h, ldh, r, ldr, norm_w, eps, workspace, k, res_out, ldres, scale, m, k, din, s);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    Problem p{workspace, w, c, m, n, k, k, ldw, ldc, NANOVLLM_GEMM_B_NK, din, dout};
    p.epi = silu_mul ? EPI_SILU_MUL : EPI_NONE;
    p.row_scale = scale;
    return launch_mfma_staged(p, s);
}

}  // namespace

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_launch(const char* kernel) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(NANOVLLM_GEMM_ELAUNCH, "%s launch failed: %s", kernel, hipGetErrorString(e));
    return NANOVLLM_GEMM_OK;
}

}  // namespace nvg

extern "C" {

int nanovllm_gemm(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                  int64_t ldc, int b_layout, int dtype_in, int dtype_out, void* stream) {
    return nvg::gemm_entry(-1, a, b, c, m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out, stream);
}

int nanovllm_gemm_with_kernel(int kernel_id, const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                              int64_t lda, int64_t ldb, int64_t ldc, int b_layout, int dtype_in, int dtype_out,
                              void* stream) {
    if (kernel_id < 0) {
        nvg::g_last_error.clear();
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel_id);
    }
    return nvg::gemm_entry(kernel_id, a, b, c, m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out, stream);
}

int nanovllm_gemm_select(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int b_layout,
                         int dtype_in, int dtype_out, int aligned16) {
    nvg::g_last_error.clear();
    const int rc = nvg::validate(m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    return nvg::select(m, n, k, lda, ldb, b_layout, dtype_in, aligned16);
}

int nanovllm_gemm_kernel_supports(int kernel_id, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                                  int64_t ldc, int b_layout, int dtype_in, int dtype_out, int aligned16) {
    nvg::g_last_error.clear();
    if (nvg::validate(m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out) != NANOVLLM_GEMM_OK) return 0;
    return nvg::supports(kernel_id, m, n, k, lda, ldb, b_layout, dtype_in, aligned16) ? 1 : 0;
}

const char* nanovllm_gemm_kernel_name(int kernel_id) {
    switch (kernel_id) {
        case NANOVLLM_GEMM_KERNEL_FP32_NAIVE: return "fp32_naive";
        case NANOVLLM_GEMM_KERNEL_FP32_TILED: return "fp32_tiled";
        case NANOVLLM_GEMM_KERNEL_MFMA_DIRECT: return "mfma_direct";
        case NANOVLLM_GEMM_KERNEL_MFMA_STAGED: return "mfma_staged";
        case NANOVLLM_GEMM_KERNEL_SPLITK_DECODE: return "splitk_decode";
        case NANOVLLM_GEMM_KERNEL_GEMV_DECODE: return "gemv_decode";
        default: return "unknown";
    }
}

int nanovllm_gemm_silu_mul(const void* a, const void* w, void* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                           int64_t ldw, int64_t ldc, int dtype_in, int dtype_out, void* stream) {
    return nvg::silu_mul_entry(-1, a, w, c, m, n, k, lda, ldw, ldc, dtype_in, dtype_out, stream);
}

int nanovllm_gemm_silu_mul_with_kernel(int kernel_id, const void* a, const void* w, void* c, int64_t m, int64_t n,
                                       int64_t k, int64_t lda, int64_t ldw, int64_t ldc, int dtype_in, int dtype_out,
                                       void* stream) {
    if (kernel_id < 0 || kernel_id >= NANOVLLM_GEMM_KERNEL_COUNT) {
        nvg::g_last_error.clear();
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel_id);
    }
    return nvg::silu_mul_entry(kernel_id, a, w, c, m, n, k, lda, ldw, ldc, dtype_in, dtype_out, stream);
}

int nanovllm_gemm_silu_mul_select(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw, int64_t ldc,
                                  int dtype_in, int dtype_out, int aligned16) {
    nvg::g_last_error.clear();
    const int rc = nvg::validate_silu_mul(m, n, k, lda, ldw, ldc, dtype_in, dtype_out);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    return nvg::select_silu_mul(m, n, k, lda, ldw, aligned16);
}

int64_t nanovllm_gemm_argmax_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw,
                                             int dtype_in) {
    nvg::g_last_error.clear();
    const int rc = nvg::validate_argmax(m, n, k, lda, ldw, dtype_in);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    return nvg::argmax_workspace_bytes(m, n);
}

int nanovllm_gemm_argmax(const void* a, const void* w, int64_t* tokens, float* max_logits, int64_t m, int64_t n,
                         int64_t k, int64_t lda, int64_t ldw, int dtype_in, int logit_dtype, void* workspace,
                         int64_t workspace_bytes, void* stream) {
    return nvg::argmax_entry(-1, a, w, tokens, max_logits, m, n, k, lda, ldw, dtype_in, logit_dtype, workspace,
                             workspace_bytes, stream);
}

int nanovllm_gemm_argmax_with_kernel(int kernel_id, const void* a, const void* w, int64_t* tokens,
                                     float* max_logits, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw,
                                     int dtype_in, int logit_dtype, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
    if (kernel_id < 0 || kernel_id >= NANOVLLM_GEMM_KERNEL_COUNT) {
        nvg::g_last_error.clear();
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel_id);
    }
    return nvg::argmax_entry(kernel_id, a, w, tokens, max_logits, m, n, k, lda, ldw, dtype_in, logit_dtype,
                             workspace, workspace_bytes, stream);
}

int nanovllm_gemm_argmax_noalloc(const void* a, const void* w, int64_t* tokens, float* max_logits, int64_t m,
                                 int64_t n, int64_t k, int64_t lda, int64_t ldw, int dtype_in, int logit_dtype,
                                 void* stream) {
    nvg::g_last_error.clear();
    int rc = nvg::validate_argmax(m, n, k, lda, ldw, dtype_in);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    rc = nvg::validate_logit_dtype(dtype_in, logit_dtype);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    const int64_t need = nvg::argmax_workspace_bytes(m, n);
    if (need > nvg::kArgmaxScratchBytes)
        return nvg::set_error(NANOVLLM_GEMM_EINVAL,
                              "argmax_noalloc: this problem needs %lld bytes of scratch (m=%lld n=%lld), above the "
                              "%lld bytes the library holds per device; call nanovllm_gemm_argmax with a workspace",
                              (long long)need, (long long)m, (long long)n, (long long)nvg::kArgmaxScratchBytes);
    if (m == 0) return NANOVLLM_GEMM_OK;
    void* scratch = nullptr;
    rc = nvg::argmax_scratch(static_cast<hipStream_t>(stream), &scratch);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    return nvg::argmax_entry(-1, a, w, tokens, max_logits, m, n, k, lda, ldw, dtype_in, logit_dtype, scratch,
                             nvg::kArgmaxScratchBytes, stream);
}

int nanovllm_gemm_sample(const void* a, const void* w, const float* temperatures, uint64_t seed, uint64_t offset,
                         int64_t* tokens, float* scores, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw,
                         int dtype_in, int logit_dtype, void* workspace, int64_t workspace_bytes, void* stream) {
    const nvg::SampleArgs sa{temperatures, seed, offset};
    return nvg::argmax_entry(-1, a, w, tokens, scores, m, n, k, lda, ldw, dtype_in, logit_dtype, workspace,
                             workspace_bytes, stream, &sa);
}

int nanovllm_gemm_sample_with_kernel(int kernel_id, const void* a, const void* w, const float* temperatures,
                                     uint64_t seed, uint64_t offset, int64_t* tokens, float* scores, int64_t m,
                                     int64_t n, int64_t k, int64_t lda, int64_t ldw, int dtype_in, int logit_dtype,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
    if (kernel_id < 0 || kernel_id >= NANOVLLM_GEMM_KERNEL_COUNT) {
        nvg::g_last_error.clear();
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel_id);
    }
    const nvg::SampleArgs sa{temperatures, seed, offset};
    return nvg::argmax_entry(kernel_id, a, w, tokens, scores, m, n, k, lda, ldw, dtype_in, logit_dtype, workspace,
                             workspace_bytes, stream, &sa);
}

int nanovllm_gemm_argmax_select(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldw, int dtype_in,
                                int aligned16) {
    nvg::g_last_error.clear();
    const int rc = nvg::validate_argmax(m, n, k, lda, ldw, dtype_in);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    return nvg::select_argmax(m, k, lda, ldw, aligned16);
}

int64_t nanovllm_gemm_gated_workspace_bytes(int64_t m, int64_t k, int64_t group, int dtype_in) {
    nvg::g_last_error.clear();
    const int rc = nvg::validate_prologue_dtypes(dtype_in, dtype_in, "gemm_gated");
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m < 0 || k < 1 || group < 1 || k % group != 0)
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "need m >= 0, k >= 1 and a group dividing k (m=%lld k=%lld "
                              "group=%lld)", (long long)m, (long long)k, (long long)group);
    return nvg::gated_workspace_bytes(m, k);
}

int nanovllm_gemm_gated(const void* a, const void* gate, const void* w, void* c, int64_t m, int64_t n, int64_t k,
                        int64_t lda, int64_t ldg, int64_t group, int64_t group_stride, int64_t ldw, int64_t ldc,
                        int dtype_in, int dtype_out, void* workspace, int64_t workspace_bytes, void* stream) {
    return nvg::gated_entry(-1, a, gate, w, c, m, n, k, lda, ldg, group, group_stride, ldw, ldc, dtype_in, dtype_out,
                            workspace, workspace_bytes, stream);
}

int nanovllm_gemm_gated_with_kernel(int kernel_id, const void* a, const void* gate, const void* w, void* c,
                                    int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldg, int64_t group,
                                    int64_t group_stride, int64_t ldw, int64_t ldc, int dtype_in, int dtype_out,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
    if (kernel_id < 0 || kernel_id >= NANOVLLM_GEMM_KERNEL_COUNT) {
        nvg::g_last_error.clear();
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel_id);
    }
    return nvg::gated_entry(kernel_id, a, gate, w, c, m, n, k, lda, ldg, group, group_stride, ldw, ldc, dtype_in,
                            dtype_out, workspace, workspace_bytes, stream);
}

int nanovllm_sigmoid_gate(const void* a, const void* gate, void* out, int64_t m, int64_t k, int64_t lda,
                          int64_t ldg, int64_t group, int64_t group_stride, int64_t ldo, int dtype, void* stream) {
    nvg::g_last_error.clear();
    int rc = nvg::validate_gated(m, 0, k, lda, ldg, group, group_stride, k, 1, dtype, dtype);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (ldo < k) return nvg::set_error(NANOVLLM_GEMM_EINVAL, "ldo (%lld) must be >= k (%lld)", (long long)ldo,
                                       (long long)k);
    if (m == 0) return NANOVLLM_GEMM_OK;
    if (a == nullptr || gate == nullptr || out == nullptr)
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "a, gate and out must be non-null device pointers");
    const int al = nvg::aligned16_ptr(a) && nvg::aligned16_ptr(gate) && nvg::aligned16_ptr(out);
    if (!nvg::gated_vector_ok(k, lda, ldg, group, group_stride, k, al) || ldo % 8 != 0)
        return nvg::set_error(NANOVLLM_GEMM_EUNSUPPORTED,
                              "sigmoid_gate needs 16-byte aligned a, gate and out with k, lda, ldg, group, "
                              "group_stride and ldo multiples of 8");
    return nvg::launch_gate_prologue(a, lda, gate, ldg, group, group_stride, out, ldo, m, k, dtype,
                                     static_cast<hipStream_t>(stream));
}

int64_t nanovllm_gemm_add_rmsnorm_workspace_bytes(int64_t m, int64_t k, int dtype_in) {
    nvg::g_last_error.clear();
    const int rc = nvg::validate_add_norm_dtypes(dtype_in, dtype_in);
    if (rc != NANOVLLM_GEMM_OK) return rc;
    if (m < 0 || k < 1)
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "need m >= 0 and k >= 1 (m=%lld k=%lld)", (long long)m,
                              (long long)k);
    return nvg::add_norm_workspace_bytes(m, k);
}

int nanovllm_gemm_add_rmsnorm(const void* h, const void* residual, const void* norm_weight, float eps, const void* w,
                              void* c, void* residual_out, int64_t m, int64_t n, int64_t k, int64_t ldh, int64_t ldr,
                              int64_t ldw, int64_t ldc, int64_t ldres, int silu_mul, int dtype_in, int dtype_out,
                              void* workspace, int64_t workspace_bytes, void* stream) {
    return nvg::add_norm_entry(-1, h, residual, norm_weight, eps, w, c, residual_out, m, n, k, ldh, ldr, ldw, ldc,
                               ldres, silu_mul, dtype_in, dtype_out, workspace, workspace_bytes, stream);
}

int nanovllm_gemm_add_rmsnorm_with_kernel(int kernel_id, const void* h, const void* residual,
                                          const void* norm_weight, float eps, const void* w, void* c,
                                          void* residual_out, int64_t m, int64_t n, int64_t k, int64_t ldh,
                                          int64_t ldr, int64_t ldw, int64_t ldc, int64_t ldres, int silu_mul,
                                          int dtype_in, int dtype_out, void* workspace, int64_t workspace_bytes,
                                          void* stream) {
    if (kernel_id < 0 || kernel_id >= NANOVLLM_GEMM_KERNEL_COUNT) {
        nvg::g_last_error.clear();
        return nvg::set_error(NANOVLLM_GEMM_EINVAL, "unknown kernel id %d", kernel_id);
    }
    return nvg::add_norm_entry(kernel_id, h, residual, norm_weight, eps, w, c, residual_out, m, n, k, ldh, ldr, ldw,
                               ldc, ldres, silu_mul, dtype_in, dtype_out, workspace, workspace_bytes, stream);
}

const char* nanovllm_gemm_last_error(void) { return nvg::g_last_error.c_str(); }

int nanovllm_gemm_version(void) { return (2 << 16) | 0; }

}  // extern "C"
