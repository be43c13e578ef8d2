// The A prologues as kernels of their own, for problems the fused decode
// kernel does not take (M > 32): they write the GEMM operand to a buffer,
// which mfma_staged then reads.  Both use the element functions of the fused
// path (gate8, add_norm8), so an element of the operand is the same bits
// either way.
//   * gate_prologue_kernel: out = round(a * round(sigmoid(g))), the output
//     gate of Qwen3.5 gated attention (nanovllm/models/qwen3_5.py:95),
//     with the gate read through the head-strided view q_proj produces
//     (qwen3_5.py:81-86: element (i, k) at g[i ldg + (k / group) stride +
//     k % group]);
//   * add_norm_prologue_kernel: residual add and zero-centred RMSNorm
//     (nanovllm/layers/layernorm.py:131-142): s = h + r in fp32, writes
//     round(s) (the new residual), round(s (1 + w)) (the GEMM operand) and
//     rsqrt(mean s^2 + eps) per row, which the GEMM applies to its output
//     rows before rounding.
#include "gemm_common.hpp"

namespace nvg {
namespace {

constexpr int kProThreads = 256;

// One thread per 16-byte chunk (8 elements) of the output, grid-stride.
template <int DT>
__global__ __launch_bounds__(kProThreads) void gate_prologue_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ g, int64_t ldg, int64_t group,
    int64_t group_stride, uint16_t* __restrict__ out, int64_t ldo, int64_t m, int64_t k) {
    const int64_t chunks = k / 8;
    const int64_t total = m * chunks;
    for (int64_t e = int64_t(blockIdx.x) * kProThreads + threadIdx.x; e < total;
         e += int64_t(gridDim.x) * kProThreads) {
        const int64_t i = e / chunks;
        const int64_t kc = (e - i * chunks) * 8;
        const u32x4_t av = load16(a + i * lda + kc);
        const u32x4_t gv = load16(g + i * ldg + (kc / group) * group_stride + kc % group);
        *reinterpret_cast<u32x4_t*>(out + i * ldo + kc) = gate8<DT>(av, gv);
    }
}

// One workgroup per row.  Thread t takes chunks t, t + 256, ...; the sum of
// squares is added in a fixed order (per thread, a butterfly over the wave,
// then the four waves in order), so the scale does not depend on timing.
template <int DT>
__global__ __launch_bounds__(kProThreads) void add_norm_prologue_kernel(
    const uint16_t* __restrict__ h, int64_t ldh, const uint16_t* __restrict__ r, int64_t ldr,
    const uint16_t* __restrict__ w, float eps, uint16_t* __restrict__ y, int64_t ldy,
    uint16_t* __restrict__ res, int64_t ldres, float* __restrict__ scale, int64_t k) {
    const int64_t i = blockIdx.x;
    float ss = 0.0f;
    for (int64_t kc = int64_t(threadIdx.x) * 8; kc < k; kc += kProThreads * 8) {
        u32x4_t rv;
        const u32x4_t yv = add_norm8<DT>(load16(h + i * ldh + kc), load16(r + i * ldr + kc), load16(w + kc), ss, rv);
        *reinterpret_cast<u32x4_t*>(y + i * ldy + kc) = yv;
        *reinterpret_cast<u32x4_t*>(res + i * ldres + kc) = rv;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    __shared__ float wave_sum[kProThreads / 64];
    if ((threadIdx.x & 63) == 0) wave_sum[threadIdx.x >> 6] = ss;
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = wave_sum[0];
#pragma unroll
        for (int wv = 1; wv < kProThreads / 64; ++wv) total += wave_sum[wv];
        scale[i] = norm_scale(total, k, eps);
    }
}

}  // namespace

int launch_gate_prologue(const void* a, int64_t lda, const void* g, int64_t ldg, int64_t group,
                         int64_t group_stride, void* out, int64_t ldo, int64_t m, int64_t k, int dtype,
                         hipStream_t s) {
    const int64_t chunks = m * (k / 8);
    if (chunks == 0) return NANOVLLM_GEMM_OK;
    const int64_t want = (chunks + kProThreads - 1) / kProThreads;
    const int64_t blocks = want < (int64_t(1) << 20) ? want : (int64_t(1) << 20);   // grid-stride beyond
    const dim3 grid(static_cast<uint32_t>(blocks)), block(kProThreads);
    const auto* ap = static_cast<const uint16_t*>(a);
    const auto* gp = static_cast<const uint16_t*>(g);
    auto* op = static_cast<uint16_t*>(out);
    if (dtype == NANOVLLM_GEMM_BF16)
        hipLaunchKernelGGL(gate_prologue_kernel<NANOVLLM_GEMM_BF16>, grid, block, 0, s, ap, lda, gp, ldg, group,
                           group_stride, op, ldo, m, k);
    else
        hipLaunchKernelGGL(gate_prologue_kernel<NANOVLLM_GEMM_F16>, grid, block, 0, s, ap, lda, gp, ldg, group,
                           group_stride, op, ldo, m, k);
    return check_launch("gate_prologue");
}

int launch_add_norm_prologue(const void* h, int64_t ldh, const void* r, int64_t ldr, const void* w, float eps,
                             void* y, int64_t ldy, void* res, int64_t ldres, float* scale, int64_t m, int64_t k,
                             int dtype, hipStream_t s) {
    if (m == 0) return NANOVLLM_GEMM_OK;
    if (m > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "add_norm_prologue: too many rows");
    const dim3 grid(static_cast<uint32_t>(m)), block(kProThreads);
    const auto* hp = static_cast<const uint16_t*>(h);
    const auto* rp = static_cast<const uint16_t*>(r);
    const auto* wp = static_cast<const uint16_t*>(w);
    auto* yp = static_cast<uint16_t*>(y);
    auto* resp = static_cast<uint16_t*>(res);
    if (dtype == NANOVLLM_GEMM_BF16)
        hipLaunchKernelGGL(add_norm_prologue_kernel<NANOVLLM_GEMM_BF16>, grid, block, 0, s, hp, ldh, rp, ldr, wp,
                           eps, yp, ldy, resp, ldres, scale, k);
    else
        hipLaunchKernelGGL(add_norm_prologue_kernel<NANOVLLM_GEMM_F16>, grid, block, 0, s, hp, ldh, rp, ldr, wp,
                           eps, yp, ldy, resp, ldres, scale, k);
    return check_launch("add_norm_prologue");
}

}  // namespace nvg
