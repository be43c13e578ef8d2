// Final step of the greedy LM head (EPI_ARGMAX): each workgroup of the GEMM
// left one key per row of A (argmax_key of its best column); this kernel
// takes the maximum key of each row over all workgroups and decodes it into
// the token id and its logit.  It stands in for Sampler's greedy branch,
// float_logits.argmax(dim=-1) (nanovllm/layers/sampler.py:8-21), which
// reads back the [M, vocab] fp32 logits the GEMM wrote.
#include <mutex>

#include "gemm_common.hpp"

namespace nvg {
namespace {

// Scratch of the no-allocation greedy head (nanovllm_gemm_argmax_noalloc):
// the [m, blocks] partial keys live in this file-scope device array instead
// of a caller workspace.  Each device that runs the entry point holds its
// own copy, at its own address, until the process ends.  In host code the
// array's name is only a stand-in for the symbol; kernels get the device
// address that hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint64_t scratch[kArgmaxScratchBytes / sizeof(uint64_t)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// One workgroup per row; a row's keys are contiguous ([m, blocks]).  Each
// thread issues kFinalizeUnroll independent loads per round, so up to 10240
// keys (the ~9500 of a 151936-entry vocabulary at 16 columns per
// workgroup) take one round of memory latency.
constexpr int kFinalizeThreads = 1024;
constexpr int kFinalizeUnroll = 10;

__global__ __launch_bounds__(kFinalizeThreads) void argmax_finalize_kernel(
    const uint64_t* __restrict__ keys, int64_t blocks, int64_t m, int64_t* __restrict__ tokens,
    float* __restrict__ logits) {
    __shared__ uint64_t best_of_wave[kFinalizeThreads / 64];
    const int64_t row = blockIdx.x;
    const uint64_t* rk = keys + row * blocks;
    uint64_t best = 0;
    for (int64_t b0 = threadIdx.x; b0 < blocks; b0 += kFinalizeThreads * kFinalizeUnroll) {
        uint64_t k[kFinalizeUnroll];
#pragma unroll
        for (int u = 0; u < kFinalizeUnroll; ++u) {
            const int64_t b = b0 + int64_t(u) * kFinalizeThreads;
            k[u] = b < blocks ? rk[b] : 0;
        }
#pragma unroll
        for (int u = 0; u < kFinalizeUnroll; ++u) best = k[u] > best ? k[u] : best;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = (uint64_t(uint32_t(__shfl_xor(int(best >> 32), off))) << 32) |
                           uint64_t(uint32_t(__shfl_xor(int(best & 0xFFFFFFFFu), off)));
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) best_of_wave[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int wv = 1; wv < kFinalizeThreads / 64; ++wv) best = best_of_wave[wv] > best ? best_of_wave[wv] : best;
        tokens[row] = int64_t(0xFFFFFFFFu - uint32_t(best & 0xFFFFFFFFu));
        if (logits != nullptr) {
            const uint32_t ordered = uint32_t(best >> 32);
            const uint32_t bits = (ordered & 0x80000000u) ? (ordered & 0x7FFFFFFFu) : ~ordered;
            logits[row] = __builtin_bit_cast(float, bits);
        }
    }
}

}  // namespace

int argmax_scratch(hipStream_t stream, void** ptr) {
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess)
        return set_error(NANOVLLM_GEMM_ELAUNCH, "argmax_noalloc: cannot find the stream's device");
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(NANOVLLM_GEMM_ELAUNCH, "argmax_noalloc: device %d beyond the %d this library tracks",
                         int(dev), kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        // Resolved once per device, with that device current: every device
        // has its own copy of the array.
        int prev = 0;
        if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(dev) != hipSuccess)
            return set_error(NANOVLLM_GEMM_ELAUNCH, "argmax_noalloc: cannot select device %d", int(dev));
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t back = hipSetDevice(prev);
        if (err != hipSuccess || p == nullptr)
            return set_error(NANOVLLM_GEMM_ELAUNCH, "argmax_noalloc: hipGetSymbolAddress failed on device %d: %s",
                             int(dev), hipGetErrorString(err));
        if (back != hipSuccess)
            return set_error(NANOVLLM_GEMM_ELAUNCH, "argmax_noalloc: cannot restore device %d", prev);
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return NANOVLLM_GEMM_OK;
}

int launch_argmax_finalize(const uint64_t* keys, int64_t blocks, int64_t m, int64_t* tokens, float* logits,
                           hipStream_t s) {
    if (m > INT32_MAX) return set_error(NANOVLLM_GEMM_EINVAL, "argmax: too many rows");
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3(static_cast<uint32_t>(m)), dim3(kFinalizeThreads), 0, s, keys,
                       blocks, m, tokens, logits);
    return check_launch("argmax_finalize");
}

}  // namespace nvg
