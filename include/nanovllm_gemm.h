/*
 * nanovllm_gemm.h — C ABI of the MI355X (gfx950) shape-aware GEMM library.
 *
 * One library, libnanovllm_gemm.so, built by hipcc for gfx950.  Every entry
 * point takes plain device pointers, sizes and an opaque HIP stream; there
 * are no torch types in any signature and no C++ exception crosses the
 * boundary.  Errors come back as negative return codes, with a thread-local
 * message from nanovllm_gemm_last_error().
 *
 * Problem computed by every GEMM entry point (row-major, fp32 accumulate):
 *
 *     C[m, n] = sum_k A[m, k] * B(k, n)
 *
 *   A  : [M, K] row-major, element (m, k) at a[m * lda + k]
 *   B  : b_layout == NANOVLLM_GEMM_B_NK: W[N, K] row-major (the nn.Linear
 *        weight layout), B(k, n) = b[n * ldb + k]
 *        b_layout == NANOVLLM_GEMM_B_KN: B[K, N] row-major,
 *        B(k, n) = b[k * ldb + n]
 *   C  : [M, N] row-major, element (m, n) at c[m * ldc + n]
 *
 * Supported dtype pairs (in -> out): f32->f32, f16->{f16,f32},
 * bf16->{bf16,f32}.  A and B share the input dtype.  Narrow outputs are the
 * round-to-nearest-even image of the fp32 accumulator.
 *
 * Reference interfaces these replace (paths relative to the reference repo):
 *   - cuda_kernels/gemm/src/gemm_bench.cu:80-196   wmma_direct_kernel / wmma_staged_kernel
 *     launched at :349-369 with B[K,N] and FP32 output;
 *   - cuda_kernels/gemm/src/gemm_wmma.cu:34-207    scalar / WMMA / staged kernels, B = W[N,K];
 *   - cuda_kernels/gemm/src/gemm_tiled.cu:36-202   FP32 naive / tiled / register-tiled kernels;
 *   - cuda_kernels/gemm/src/gemm.cu:7-15           FP32 one-thread-per-output kernel;
 *   - cuda_kernels/gemm/src/gemm_bench.cu:252-282  supports_wmma / choose_path / path_name;
 *   - nanovllm/layers/linear.py:51,73,153 and nanovllm/layers/embed_head.py:61
 *     F.linear(x, W) call sites (W[N,K], the NK layout here).
 */
#ifndef NANOVLLM_GEMM_H
#define NANOVLLM_GEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types.  Values are part of the ABI. */
enum {
    NANOVLLM_GEMM_F32 = 0,
    NANOVLLM_GEMM_F16 = 1,
    NANOVLLM_GEMM_BF16 = 2
};

/* Layout of the second operand.  Values are part of the ABI. */
enum {
    NANOVLLM_GEMM_B_NK = 0, /* W[N, K] row-major (nn.Linear weight)   */
    NANOVLLM_GEMM_B_KN = 1  /* B[K, N] row-major (gemm_bench.cu:103)  */
};

/* Kernel identifiers returned by nanovllm_gemm_select().  The ladder
 * mirrors the reference's rungs; none of them is a vendor-library call.
 *   FP32_NAIVE     one thread per output            (gemm.cu:7-15, gemm_tiled.cu:36-51)
 *   FP32_TILED     LDS-tiled fp32 MFMA kernel       (gemm_tiled.cu:56-202)
 *   MFMA_DIRECT    one wave per 32x32 C tile, operands straight from
 *                  global memory, any shape          (gemm_bench.cu:80-115, gemm_wmma.cu:56-104)
 *   MFMA_STAGED    LDS multi-buffered macro-tile MFMA kernel for
 *                  prefill-shaped problems on W[N,K] and on B[K,N] with N a
 *                  multiple of 8 (B's k-rows copied to LDS as they lie,
 *                  read back transposed)
 *                                                    (gemm_bench.cu:117-196, gemm_wmma.cu:116-207)
 *   SPLITK_DECODE  split-K wavefront-reduction kernel for M <= 32 (the
 *                  plain GEMM and the fused SiLU-and-mul up to M = 64 below
 *                  65536 W rows; B[K,N] up to M = 64, 64 columns per
 *                  workgroup, read back transposed) that streams W once,
 *                  copied to LDS in whole 128-byte lines; selected for
 *                  B[K,N] up to M = 32 (M = 64 on N <= 4096) and, on W[N,K],
 *                  for 2 <= M <= 32, for
 *                  M == 1 when W is larger than 64 MiB (LM head), for
 *                  33 <= M <= 64 when N <= 4096 (or N <= 10240 with
 *                  K <= 1024), and for the fused SiLU-and-mul at every
 *                  M <= 32 and at 33 <= M <= 64 with 2n <= 16384
 *                                                    (replaces the cuBLAS fallback of
 *                                                     gemm_bench.cu:260-273 for decode shapes)
 *   GEMV_DECODE    M == 1: one wave per W row, coalesced 16-byte streaming,
 *                  VALU dot products; selected when W is at most 64 MiB
 *                                                    (the qwen35_decode_qkv shape of
 *                                                     gemm_bench.cu:46, cuBLAS there)
 */
enum {
    NANOVLLM_GEMM_KERNEL_FP32_NAIVE = 0,
    NANOVLLM_GEMM_KERNEL_FP32_TILED = 1,
    NANOVLLM_GEMM_KERNEL_MFMA_DIRECT = 2,
    NANOVLLM_GEMM_KERNEL_MFMA_STAGED = 3,
    NANOVLLM_GEMM_KERNEL_SPLITK_DECODE = 4,
    NANOVLLM_GEMM_KERNEL_GEMV_DECODE = 5,
    NANOVLLM_GEMM_KERNEL_COUNT = 6
};

/* Return codes. */
enum {
    NANOVLLM_GEMM_OK = 0,
    NANOVLLM_GEMM_EINVAL = -1,      /* bad size, stride, pointer or enum  */
    NANOVLLM_GEMM_EUNSUPPORTED = -2, /* dtype pair / kernel cannot run it  */
    NANOVLLM_GEMM_ELAUNCH = -3      /* HIP reported an error at launch    */
};

/*
 * Shape-aware GEMM.  Picks the kernel with nanovllm_gemm_select() and
 * enqueues it on `stream` (a hipStream_t; NULL is the default stream).
 * Asynchronous: no host synchronisation, no allocation, capturable into a
 * HIP graph.  Replaces choose_path + the launch lambdas of
 * gemm_bench.cu:260-273, 349-369 and the F.linear call of linear.py:51.
 * Returns NANOVLLM_GEMM_OK or a negative code.
 */
int nanovllm_gemm(const void* a, const void* b, void* c,
                  int64_t m, int64_t n, int64_t k,
                  int64_t lda, int64_t ldb, int64_t ldc,
                  int b_layout, int dtype_in, int dtype_out,
                  void* stream);

/*
 * Same problem, forced onto one kernel of the ladder (for parity tests of
 * every rung and for the benchmark ladder, like gemm_bench.cu:396-416
 * timing direct and staged side by side).  Returns
 * NANOVLLM_GEMM_EUNSUPPORTED when that kernel cannot run the problem
 * (checked by nanovllm_gemm_kernel_supports()).
 */
int nanovllm_gemm_with_kernel(int kernel_id,
                              const void* a, const void* b, void* c,
                              int64_t m, int64_t n, int64_t k,
                              int64_t lda, int64_t ldb, int64_t ldc,
                              int b_layout, int dtype_in, int dtype_out,
                              void* stream);

/*
 * Shape-selection table: the kernel nanovllm_gemm() would launch for this
 * problem, given that the pointers are 16-byte aligned when `aligned16` is
 * non-zero.  Pure host function; callable without a GPU.  Replaces
 * supports_wmma + choose_path (gemm_bench.cu:252-273).  Returns a kernel id
 * or a negative code for an invalid problem.
 */
int nanovllm_gemm_select(int64_t m, int64_t n, int64_t k,
                         int64_t lda, int64_t ldb, int64_t ldc,
                         int b_layout, int dtype_in, int dtype_out,
                         int aligned16);

/* 1 when `kernel_id` can run the problem, else 0.  Pure host function. */
int nanovllm_gemm_kernel_supports(int kernel_id,
                                  int64_t m, int64_t n, int64_t k,
                                  int64_t lda, int64_t ldb, int64_t ldc,
                                  int b_layout, int dtype_in, int dtype_out,
                                  int aligned16);

/*
 * Fused gate/up projection and SiLU-and-mul of the Qwen3.5 MLP:
 *
 *     c[m, j] = silu(sum_k a[m,k] w[j,k]) * sum_k a[m,k] w[n + j, k],  j < n
 *
 * with w = [W_gate; W_up], 2n rows in the W[N,K] layout (the weight of the
 * MergedColumnParallelLinear gate_up_proj, nanovllm/layers/linear.py:76-97)
 * and silu(x) = x / (1 + e^-x).  Both sums accumulate in fp32; silu and the
 * product are evaluated in fp32 and rounded once to dtype_out (f16->{f16,f32},
 * bf16->{bf16,f32}).  Replaces gate_up_proj followed by SiluAndMul
 * (nanovllm/models/qwen3_5.py:117, nanovllm/layers/activation.py:8-11),
 * which writes and re-reads the [m, 2n] projection.  Needs the vector path
 * (16-byte aligned a and w, k, lda and ldw multiples of 8); otherwise
 * NANOVLLM_GEMM_EUNSUPPORTED.  Asynchronous, no allocation, capturable.
 */
int nanovllm_gemm_silu_mul(const void* a, const void* w, void* c,
                           int64_t m, int64_t n, int64_t k,
                           int64_t lda, int64_t ldw, int64_t ldc,
                           int dtype_in, int dtype_out,
                           void* stream);

/* The fused problem forced onto one kernel (mfma_staged, splitk_decode for
 * m <= 32, gemv_decode for m == 1), as nanovllm_gemm_with_kernel does for
 * the plain GEMM (gemm_bench.cu:396-416 pattern). */
int nanovllm_gemm_silu_mul_with_kernel(int kernel_id,
                                       const void* a, const void* w, void* c,
                                       int64_t m, int64_t n, int64_t k,
                                       int64_t lda, int64_t ldw, int64_t ldc,
                                       int dtype_in, int dtype_out,
                                       void* stream);

/* Kernel id nanovllm_gemm_silu_mul() would launch (or a negative code).
 * Pure host function, like nanovllm_gemm_select (gemm_bench.cu:252-273). */
int nanovllm_gemm_silu_mul_select(int64_t m, int64_t n, int64_t k,
                                  int64_t lda, int64_t ldw, int64_t ldc,
                                  int dtype_in, int dtype_out, int aligned16);

/*
 * Greedy token of an LM head without its logits:
 *
 *     tokens[i] = argmax_j L(sum_k a[i,k] w[j,k]),   j < n
 *
 * fp32 accumulation, first index on ties, NaN above every number (the
 * rule of torch.argmax), token ids as int64.  L is the logit the head
 * ranks, chosen by logit_dtype:
 *   - logit_dtype == dtype_in: the fp32 sum rounded to nearest even in the
 *     input type, i.e. the logits ParallelLMHead's F.linear returns in the
 *     model dtype (nanovllm/layers/embed_head.py:61), which Sampler ranks
 *     after .float() (nanovllm/layers/sampler.py:15, 21).  This is the
 *     reference's greedy token; equal rounded logits go to the first index;
 *   - logit_dtype == NANOVLLM_GEMM_F32: the fp32 sum itself (finer ranking
 *     than the reference; opt-in).
 * Any other logit_dtype is NANOVLLM_GEMM_EINVAL.  max_logits[i] (optional,
 * may be NULL) receives L of the token as fp32.  Replaces the [m, n] logits
 * of ParallelLMHead followed by the greedy branch of Sampler,
 * float_logits.argmax(dim=-1) (nanovllm/layers/sampler.py:8-21).
 * `workspace` (8-byte aligned, device memory, contents scratch) must hold
 * nanovllm_gemm_argmax_workspace_bytes() bytes; one call launches the GEMM
 * pass and a small reduction pass on `stream`.  Inputs f16 or bf16 on the
 * vector path (16-byte aligned a and w, k, lda and ldw multiples of 8).
 */
int nanovllm_gemm_argmax(const void* a, const void* w,
                         int64_t* tokens, float* max_logits,
                         int64_t m, int64_t n, int64_t k,
                         int64_t lda, int64_t ldw, int dtype_in, int logit_dtype,
                         void* workspace, int64_t workspace_bytes,
                         void* stream);

/*
 * nanovllm_gemm_argmax without a workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  It has no counterpart in the
 * reference.  The partial keys go to a scratch array the library holds in
 * device memory: 8 MiB per device (1 << 23 bytes), enough for every
 * problem whose nanovllm_gemm_argmax_workspace_bytes() is at most that
 * (the 151936-entry vocabulary up to m = 883: 1187 keys of 8 bytes per
 * row); larger problems return NANOVLLM_GEMM_EINVAL before anything is
 * launched.  Calls no allocator.  The first call with m >= 1 on a device
 * resolves that device's copy of the array (hipGetSymbolAddress, with the
 * stream's device made current for the call): make it before capturing a
 * HIP graph that contains this entry point.  Every call on one device
 * shares that device's array: calls that overlap on one device (two
 * streams, two threads) race and must be ordered by the caller.  Same
 * arguments and results as nanovllm_gemm_argmax otherwise.
 */
int nanovllm_gemm_argmax_noalloc(const void* a, const void* w,
                                 int64_t* tokens, float* max_logits,
                                 int64_t m, int64_t n, int64_t k,
                                 int64_t lda, int64_t ldw, int dtype_in, int logit_dtype,
                                 void* stream);

/* Workspace bytes nanovllm_gemm_argmax needs for this problem (enough for
 * any kernel that can run it), or a negative code.  Pure host function. */
int64_t nanovllm_gemm_argmax_workspace_bytes(int64_t m, int64_t n, int64_t k,
                                             int64_t lda, int64_t ldw, int dtype_in);

/* The greedy head forced onto one kernel (splitk_decode for m <= 32 or
 * mfma_staged), for parity tests of both (gemm_bench.cu:396-416 pattern). */
int nanovllm_gemm_argmax_with_kernel(int kernel_id,
                                     const void* a, const void* w,
                                     int64_t* tokens, float* max_logits,
                                     int64_t m, int64_t n, int64_t k,
                                     int64_t lda, int64_t ldw, int dtype_in, int logit_dtype,
                                     void* workspace, int64_t workspace_bytes,
                                     void* stream);

/* Kernel id nanovllm_gemm_argmax() would run its GEMM pass on (or a
 * negative code).  Pure host function (gemm_bench.cu:252-273 pattern). */
int nanovllm_gemm_argmax_select(int64_t m, int64_t n, int64_t k,
                                int64_t lda, int64_t ldw, int dtype_in,
                                int aligned16);

/*
 * Sampled LM head: Sampler.forward (nanovllm/layers/sampler.py:8-21) on the
 * logits a w^T without writing them.  Row i with temperatures[i] <= 1e-10
 * takes the greedy token, exactly as nanovllm_gemm_argmax; every other row
 * takes
 *
 *     tokens[i] = argmax_j (l[i,j] / temperatures[i] - ln E[i,j]),
 *
 * l the logits as nanovllm_gemm_argmax ranks them (logit_dtype: rounded to
 * the input type as the reference's F.linear returns them, or fp32), which
 * is the reference's argmax_j of
 * softmax(l / T)_j / E_j (the Gumbel-max form of a draw from softmax(l / T)).
 * E[i,j] = max(-ln u, 1e-10) with u = ((x >> 8) + 1) / 2^24 and x word
 * j % 4 of Philox4x32-10(counter = {j / 4, i, offset, offset >> 32},
 * key = {seed, seed >> 32}), so a (seed, offset) pair fixes every draw;
 * callers advance `offset` between steps (the reference draws fresh
 * exponentials from torch's generator on every call).  A call captured in a
 * HIP graph replays its own seed and offset.  scores[i] (optional) receives
 * the winning score (the logit on greedy rows).  temperatures: m floats in
 * device memory.  Workspace as nanovllm_gemm_argmax (same size function).
 */
int nanovllm_gemm_sample(const void* a, const void* w,
                         const float* temperatures, uint64_t seed, uint64_t offset,
                         int64_t* tokens, float* scores,
                         int64_t m, int64_t n, int64_t k,
                         int64_t lda, int64_t ldw, int dtype_in, int logit_dtype,
                         void* workspace, int64_t workspace_bytes,
                         void* stream);

/* The sampled head forced onto one kernel (splitk_decode for m <= 32 or
 * mfma_staged), for parity tests of both (gemm_bench.cu:396-416 pattern). */
int nanovllm_gemm_sample_with_kernel(int kernel_id,
                                     const void* a, const void* w,
                                     const float* temperatures, uint64_t seed, uint64_t offset,
                                     int64_t* tokens, float* scores,
                                     int64_t m, int64_t n, int64_t k,
                                     int64_t lda, int64_t ldw, int dtype_in, int logit_dtype,
                                     void* workspace, int64_t workspace_bytes,
                                     void* stream);

/* Gated-attention output projection: the output gate of Qwen3.5 gated
 * attention applied to A in front of o_proj,
 *     c = (a * sigmoid(gate)) w^T
 * replacing `output * torch.sigmoid(gate)` and `self.o_proj(...)`
 * (nanovllm/models/qwen3_5.py:95-96).  As there, sigmoid(gate) is rounded to
 * the input type and so is the product, before the GEMM accumulates in
 * fp32.  The gate is read through q_proj's head-strided view
 * (qwen3_5.py:81-86): element (i, k) at
 *     gate[i * ldg + (k / group) * group_stride + k % group]
 * (group = head_dim, group_stride = 2 head_dim for q_gate; a contiguous
 * [m, k] gate is group = group_stride = k).  For m <= 8 and group a
 * multiple of 64 the gate is applied inside the split-K decode kernel (one
 * launch, no workspace; every workgroup gates all of A, which stops paying
 * above m = 8); otherwise a gate kernel writes the gated operand to the
 * workspace (nanovllm_gemm_gated_workspace_bytes() bytes) and the GEMM the
 * selection table picks reads it.  Inputs f16 or bf16, output the input
 * type or f32, on the vector path (16-byte aligned a, gate and w; k, lda,
 * ldg, group, group_stride and ldw multiples of 8).  Asynchronous, no
 * allocation, capturable. */
int nanovllm_gemm_gated(const void* a, const void* gate, const void* w, void* c,
                        int64_t m, int64_t n, int64_t k,
                        int64_t lda, int64_t ldg, int64_t group, int64_t group_stride,
                        int64_t ldw, int64_t ldc,
                        int dtype_in, int dtype_out,
                        void* workspace, int64_t workspace_bytes,
                        void* stream);

/* Workspace bytes nanovllm_gemm_gated needs with any kernel that can run
 * the problem (the fused gate uses none: workspace may then be null), or a
 * negative code.  Pure host function. */
int64_t nanovllm_gemm_gated_workspace_bytes(int64_t m, int64_t k, int64_t group, int dtype_in);

/* The gated GEMM forced onto one kernel: splitk_decode runs the fused gate
 * (m <= 32, group % 64 == 0), any other id runs the gate kernel and that
 * GEMM kernel (gemm_bench.cu:396-416 pattern). */
int nanovllm_gemm_gated_with_kernel(int kernel_id,
                                    const void* a, const void* gate, const void* w, void* c,
                                    int64_t m, int64_t n, int64_t k,
                                    int64_t lda, int64_t ldg, int64_t group, int64_t group_stride,
                                    int64_t ldw, int64_t ldc,
                                    int dtype_in, int dtype_out,
                                    void* workspace, int64_t workspace_bytes,
                                    void* stream);

/* The gate alone: out[i, k] = round(a[i, k] * round(sigmoid(gate(i, k)))),
 * the same bits the fused path feeds its GEMM (qwen3_5.py:95).  Same layout
 * rules as nanovllm_gemm_gated; out has leading dimension ldo. */
int nanovllm_sigmoid_gate(const void* a, const void* gate, void* out,
                          int64_t m, int64_t k,
                          int64_t lda, int64_t ldg, int64_t group, int64_t group_stride,
                          int64_t ldo, int dtype, void* stream);

/* Residual add + zero-centred RMSNorm in front of a projection, replacing
 * `hidden_states, residual = norm(hidden_states, residual)` followed by the
 * projection (nanovllm/models/qwen3_5.py:157-159 and 200-203 with
 * Qwen3_5RMSNorm, nanovllm/layers/layernorm.py:131-142):
 *     s = h + residual  (fp32),  residual_out = round(s),
 *     c[i, j] = rsqrt(mean_k s[i, k]^2 + eps) * sum_k round(s[i, k] (1 + w_norm[k])) w[j, k]
 * The reference rounds s * rsqrt(...) * (1 + w_norm) to the input type and
 * then multiplies; here the per-row scale is applied to the fp32 sum, so the
 * operand is rounded before scaling (one rounding per element either way).
 * silu_mul = 1 fuses SiluAndMul as nanovllm_gemm_silu_mul does: w is
 * [W_gate; W_up] with 2n rows and c[i, j] = silu(g) u of the scaled sums.
 * For m <= 32 the add and the norm run inside the split-K decode kernel
 * (one launch, no workspace); otherwise a prologue kernel writes the
 * operand and the row scales to the workspace
 * (nanovllm_gemm_add_rmsnorm_workspace_bytes()) and mfma_staged scales its
 * output rows.  Inputs bf16 (h, residual, w_norm and w alike; f16 gets
 * NANOVLLM_GEMM_EUNSUPPORTED, because the unscaled operand s (1 + w_norm)
 * can leave f16's range where the reference's normalised one does not),
 * output bf16 or f32; 16-byte aligned h, residual, w_norm, w and
 * residual_out, with k, ldh, ldr, ldres and ldw multiples of 8.
 * Asynchronous, no allocation, capturable. */
int nanovllm_gemm_add_rmsnorm(const void* h, const void* residual, const void* norm_weight, float eps,
                              const void* w, void* c, void* residual_out,
                              int64_t m, int64_t n, int64_t k,
                              int64_t ldh, int64_t ldr, int64_t ldw, int64_t ldc, int64_t ldres,
                              int silu_mul, int dtype_in, int dtype_out,
                              void* workspace, int64_t workspace_bytes,
                              void* stream);

/* Workspace bytes nanovllm_gemm_add_rmsnorm needs with either kernel (the
 * fused norm, m <= 32, uses none: workspace may then be null), or a
 * negative code.  Pure host function. */
int64_t nanovllm_gemm_add_rmsnorm_workspace_bytes(int64_t m, int64_t k, int dtype_in);

/* nanovllm_gemm_add_rmsnorm forced onto splitk_decode (fused, m <= 32) or
 * mfma_staged (prologue kernel + row-scaled GEMM). */
int nanovllm_gemm_add_rmsnorm_with_kernel(int kernel_id,
                                          const void* h, const void* residual, const void* norm_weight, float eps,
                                          const void* w, void* c, void* residual_out,
                                          int64_t m, int64_t n, int64_t k,
                                          int64_t ldh, int64_t ldr, int64_t ldw, int64_t ldc, int64_t ldres,
                                          int silu_mul, int dtype_in, int dtype_out,
                                          void* workspace, int64_t workspace_bytes,
                                          void* stream);

/* Stable name of a kernel id ("fp32_tiled", "mfma_staged", ...), or
 * "unknown".  Mirrors path_name (gemm_bench.cu:275-282). */
const char* nanovllm_gemm_kernel_name(int kernel_id);

/* Message describing the last error on the calling thread ("" if none). */
const char* nanovllm_gemm_last_error(void);

/* Library version, (major << 16) | minor. */
int nanovllm_gemm_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NANOVLLM_GEMM_H */
