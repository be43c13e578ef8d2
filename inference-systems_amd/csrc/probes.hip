// Microbenchmarks of the MI355X ceilings the GEMM kernels are measured
// against: launch floor, streaming HBM read, LDS fragment reads, the
// global -> LDS copy paths, the bf16 MFMA rate and the shader clock under
// each load.  Built into libnanovllm_probes.so (not the GEMM library) and
// driven by `bench.py --probes`.
//
// Every probe reads only inside the buffers it is given (the host wrapper
// checks sizes before launching), writes one 32-bit value per workgroup
// into `sink` (so no load is dead code), and, from lane 0 of wave 0 of
// workgroup 0, the shader-clock counter (s_memtime) and the 100 MHz
// real-time counter (s_memrealtime) at its start and end into clocks[0..3],
// from which the host derives the clock the probe ran at.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kErr = -1;

__device__ __forceinline__ void stamp(uint64_t* clocks, int slot) {
    if (clocks != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
        const uint64_t t = __builtin_amdgcn_s_memtime();
        const uint64_t r = __builtin_amdgcn_s_memrealtime();
        clocks[2 * slot] = t;
        clocks[2 * slot + 1] = r;
    }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One global_load_lds_dwordx4: lane L copies 16 bytes from src to LDS bytes
// lds + 16 L .. + 15 (the copy instruction the GEMM kernels use).
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_address(const void* p) {
    typedef const __attribute__((address_space(3))) char* lds_ptr;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)p));
}

__device__ __forceinline__ uint32_t fold(u32x4_t v) { return v[0] ^ v[1] ^ v[2] ^ v[3]; }

// XOR of x over the wave, written by lane 0 to sink[blockIdx.x * 8 + wave].
__device__ __forceinline__ void sink_wave(uint32_t* sink, uint32_t x) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) x ^= uint32_t(__shfl_xor(int(x), d));
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 8 + (threadIdx.x >> 6)] = x;
}

__global__ void empty_kernel() {}

// Streaming read of `chunks` 16-byte chunks: lane t of the grid reads chunks
// t, t + T, ..., t + (PL - 1) T (T = threads in the grid), all PL loads
// issued before the first use.  The host makes chunks == PL * T.
template <int PL>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4_t* __restrict__ buf, uint32_t* sink,
                                                          uint64_t* clocks) {
    stamp(clocks, 0);
    const int64_t threads = int64_t(gridDim.x) * blockDim.x;
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    u32x4_t v[PL];
#pragma unroll
    for (int j = 0; j < PL; ++j) v[j] = __builtin_nontemporal_load(buf + t + j * threads);
    uint32_t x = 0;
#pragma unroll
    for (int j = 0; j < PL; ++j) x ^= fold(v[j]);
    sink_wave(sink, x);
    stamp(clocks, 1);
}

// LDS fragment reads: each of the 8 waves reads 1 KiB per ds_read_b128
// (lane L: bytes 16 L .. 16 L + 15 of one of its eight 1 KiB slots, a
// conflict-free pattern), `iters` times.  64 KiB of LDS, zeroed first.
__global__ __launch_bounds__(512) void lds_read_kernel(int iters, uint32_t* sink, uint64_t* clocks) {
    __shared__ u32x4_t lds[64 * 1024 / 16];
    for (int i = threadIdx.x; i < 64 * 1024 / 16; i += blockDim.x) lds[i] = u32x4_t{0u, 0u, 0u, uint32_t(i)};
    __syncthreads();
    stamp(clocks, 0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const u32x4_t* base = lds + wave * 512 + lane;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    for (int i = 0; i < iters; i += 8) {
        u32x4_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = base[64 * j];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= v[j];
        asm volatile("" : "+v"(acc));
    }
    sink_wave(sink, fold(acc));
    stamp(clocks, 1);
}

// Global -> LDS copies with global_load_lds_dwordx4, the GEMM kernels' copy
// instruction.  Wave w of workgroup b copies 1 KiB per instruction from
// `src` (a window of `window` bytes, 1 KiB aligned) into one of its eight
// 1 KiB LDS slots, `iters` instructions, at most INFLIGHT outstanding.  With
// READS > 0 every copy is followed by READS ds_read_b128 of 1 KiB from a
// second 64 KiB region (the fragment reads a GEMM K-step makes next to its
// copies), so the LDS serves both.
template <int INFLIGHT, int READS>
__device__ __forceinline__ u32x4_t dma_body(const char* __restrict__ src, int64_t window, int iters, u32x4_t* lds,
                                            int wave, int lane) {
    const int64_t slots = window / 1024;
    int64_t slot = (int64_t(blockIdx.x) * 8 + wave) * 37 % slots;
    const uint32_t dst0 = __builtin_amdgcn_readfirstlane(lds_address(lds) + uint32_t(wave) * 8192u);
    const u32x4_t* rd = lds + 4096 + wave * 512 + lane;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    for (int i = 0; i < iters; ++i) {
        dma16(src + slot * 1024 + lane * 16, dst0 + uint32_t(i & 7) * 1024u);
        slot = slot + 1 == slots ? 0 : slot + 1;
#pragma unroll
        for (int r = 0; r < READS; ++r) acc ^= rd[((i * READS + r) & 7) * 64];
        wait_vmcnt<INFLIGHT - 1>();
    }
    wait_vmcnt<0>();
    return acc;
}

template <int INFLIGHT, int READS>
__global__ __launch_bounds__(512) void dma_kernel(const char* __restrict__ src, int64_t window, int iters,
                                                  uint32_t* sink, uint64_t* clocks) {
    __shared__ u32x4_t lds[2 * 64 * 1024 / 16];
    stamp(clocks, 0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const u32x4_t acc = dma_body<INFLIGHT, READS>(src, window, iters, lds, wave, lane);
    __syncthreads();
    sink_wave(sink, fold(lds[wave * 512 + lane] ^ acc));
    stamp(clocks, 1);
}

// Global -> VGPR loads of the same pattern (global_load_dwordx4), folded
// into a register; with STORE the loaded chunks are also written to LDS
// with ds_write_b128 (the register-staged copy path); READS as above.
template <int INFLIGHT, int STORE, int READS>
__device__ __forceinline__ u32x4_t vload_body(const char* __restrict__ src, int64_t window, int iters, u32x4_t* lds,
                                              int wave, int lane) {
    const int64_t slots = window / 1024;
    int64_t slot = (int64_t(blockIdx.x) * 8 + wave) * 37 % slots;
    const u32x4_t* rd = lds + 4096 + wave * 512 + lane;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    for (int i = 0; i < iters; i += INFLIGHT) {
        u32x4_t v[INFLIGHT];
#pragma unroll
        for (int j = 0; j < INFLIGHT; ++j) {
            v[j] = *reinterpret_cast<const u32x4_t*>(src + slot * 1024 + lane * 16);
            slot = slot + 1 == slots ? 0 : slot + 1;
        }
#pragma unroll
        for (int j = 0; j < INFLIGHT; ++j) {
            if constexpr (STORE) lds[wave * 512 + (j & 7) * 64 + lane] = v[j];
            else acc ^= v[j];
#pragma unroll
            for (int r = 0; r < READS; ++r) acc ^= rd[((j * READS + r) & 7) * 64];
        }
        // The stores of one round are not dead (nor the loads behind them)
        // just because the next round overwrites the same LDS slots.
        asm volatile("" ::: "memory");
    }
    return acc;
}

template <int INFLIGHT, int STORE, int READS>
__global__ __launch_bounds__(512) void vload_kernel(const char* __restrict__ src, int64_t window, int iters,
                                                    uint32_t* sink, uint64_t* clocks) {
    __shared__ u32x4_t lds[2 * 64 * 1024 / 16];
    stamp(clocks, 0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    u32x4_t acc = vload_body<INFLIGHT, STORE, READS>(src, window, iters, lds, wave, lane);
    if constexpr (STORE) {
        __syncthreads();
        acc ^= lds[wave * 512 + lane];
    }
    sink_wave(sink, fold(acc));
    stamp(clocks, 1);
}

// Both copy paths at once: waves 0-3 copy with global_load_lds_dwordx4,
// waves 4-7 load into registers and write LDS with ds_write_b128 (the same
// bytes per wave), to see whether the two paths add up.
template <int INFLIGHT, int READS>
__global__ __launch_bounds__(512) void hybrid_kernel(const char* __restrict__ src, int64_t window, int iters,
                                                     uint32_t* sink, uint64_t* clocks) {
    __shared__ u32x4_t lds[2 * 64 * 1024 / 16];
    stamp(clocks, 0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    u32x4_t acc;
    if (wave < 4) acc = dma_body<INFLIGHT, READS>(src, window, iters, lds, wave, lane);
    else acc = vload_body<INFLIGHT, 1, READS>(src, window, iters, lds, wave, lane);
    __syncthreads();
    sink_wave(sink, fold(lds[wave * 512 + lane] ^ acc));
    stamp(clocks, 1);
}

// v_mfma_f32_32x32x16_bf16 back to back: CHAINS independent accumulators
// per wave, `iters` rounds (iters * CHAINS MFMAs per wave).
template <int CHAINS>
__global__ __launch_bounds__(512) void mfma_kernel(int iters, uint32_t* sink, uint64_t* clocks) {
    stamp(clocks, 0);
    const int lane = threadIdx.x & 63;
    const __bf16 one = static_cast<__bf16>(1.0f / 1024.0f);
    const __bf16 x = static_cast<__bf16>(float(lane & 7) / 8.0f);
    const bf16x8_t a = {one, one, one, one, one, one, one, one};
    const bf16x8_t b = {x, x, x, x, x, x, x, x};
    f32x16_t acc[CHAINS];
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) acc[c] = f32x16_t{};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < CHAINS; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CHAINS; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) s += acc[c][v];
    sink_wave(sink, __builtin_bit_cast(uint32_t, s));
    stamp(clocks, 1);
}

// v_mfma_f32_16x16x32_bf16 back to back: CHAINS independent accumulators
// per wave (each accumulator is 4 registers), `iters` rounds.
template <int CHAINS>
__global__ __launch_bounds__(512) void mfma16_kernel(int iters, uint32_t* sink, uint64_t* clocks) {
    stamp(clocks, 0);
    const int lane = threadIdx.x & 63;
    const __bf16 one = static_cast<__bf16>(1.0f / 1024.0f);
    const __bf16 x = static_cast<__bf16>(float(lane & 7) / 8.0f);
    const bf16x8_t a = {one, one, one, one, one, one, one, one};
    const bf16x8_t b = {x, x, x, x, x, x, x, x};
    f32x4_t acc[CHAINS];
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) acc[c] = f32x4_t{};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < CHAINS; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CHAINS; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) s += acc[c][v];
    sink_wave(sink, __builtin_bit_cast(uint32_t, s));
    stamp(clocks, 1);
}

// Output-tile writes: workgroup w writes rows [128 (w / tiles_n), +128) x
// bytes [512 (w % tiles_n), +512) of a row-major matrix with `ld` bytes per
// row (the C tiles of a 128 x 256 bf16 GEMM grid), 16 bytes per lane and
// pass, non-temporal (NT) or plain stores.
template <int NT>
__global__ __launch_bounds__(512) void write_tiles_kernel(char* __restrict__ dst, int64_t ld, int tiles_n,
                                                          uint64_t* clocks) {
    stamp(clocks, 0);
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int chunk = threadIdx.x & 31, row0 = threadIdx.x >> 5;
    const u32x4_t v = {threadIdx.x, blockIdx.x, 1u, 2u};
#pragma unroll
    for (int pass = 0; pass < 8; ++pass) {
        u32x4_t* p = reinterpret_cast<u32x4_t*>(dst + (int64_t(tm) * 128 + row0 + 16 * pass) * ld +
                                                int64_t(tn) * 512 + chunk * 16);
        if constexpr (NT) __builtin_nontemporal_store(v, p);
        else *p = v;
    }
    stamp(clocks, 1);
}

// LDS lane grouping: every wave of a 256-thread workgroup issues `iters`
// LDS instructions of W bytes per lane (reads, or writes when WRITE), lane
// L at byte offset map.off[L] of a 16 KiB region (each wave its own copy of
// the region, so writes of different waves never meet), 8 in flight before
// each wait.  Lane 0 of each workgroup's wave 0 writes the shader clocks
// the loop took to cycles[blockIdx.x]; the host divides by 4 * iters for
// the LDS cycles per instruction of the CU.  Which lanes the LDS serves in
// the same clock shows as the maps with no extra cycles.
struct LaneMap { uint32_t off[64]; };

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int W>
__device__ __forceinline__ void lds_rd(uint32_t addr, u32x4_t& v) {
    if constexpr (W == 16) {
        asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    } else if constexpr (W == 8) {
        uint64_t x;
        asm volatile("ds_read_b64 %0, %1" : "=v"(x) : "v"(addr) : "memory");
        v = u32x4_t{uint32_t(x), uint32_t(x >> 32), 0u, 0u};
    } else {
        uint32_t x;
        asm volatile("ds_read_b32 %0, %1" : "=v"(x) : "v"(addr) : "memory");
        v = u32x4_t{x, 0u, 0u, 0u};
    }
}

template <int W>
__device__ __forceinline__ void lds_wr(uint32_t addr, u32x4_t v) {
    if constexpr (W == 16) {
        asm volatile("ds_write_b128 %0, %1" :: "v"(addr), "v"(v) : "memory");
    } else if constexpr (W == 8) {
        const uint64_t x = uint64_t(v[0]) | (uint64_t(v[1]) << 32);
        asm volatile("ds_write_b64 %0, %1" :: "v"(addr), "v"(x) : "memory");
    } else {
        asm volatile("ds_write_b32 %0, %1" :: "v"(addr), "v"(v[0]) : "memory");
    }
}

template <int W, bool WRITE>
__global__ __launch_bounds__(256) void lds_map_kernel(LaneMap map, int iters, uint32_t* sink, uint64_t* cycles) {
    __shared__ u32x4_t lds[4 * 16384 / 16];
    for (int i = threadIdx.x; i < 4 * 1024; i += 256) lds[i] = u32x4_t{uint32_t(i), 0u, 0u, 0u};
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t addr = lds_address(lds) + uint32_t(wave) * 16384u + map.off[lane];
    u32x4_t acc = {0u, 0u, 0u, uint32_t(lane)};
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    for (int i = 0; i < iters; i += 8) {
        if constexpr (WRITE) {
#pragma unroll
            for (int j = 0; j < 8; ++j) lds_wr<W>(addr, acc);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            acc[0] += 1u;
        } else {
            u32x4_t v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) lds_rd<W>(addr, v[j]);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int j = 0; j < 8; ++j) acc ^= v[j];
        }
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    __syncthreads();
    if (threadIdx.x == 0) cycles[blockIdx.x] = t1 - t0;
    sink_wave(sink, fold(acc));
}
#pragma clang diagnostic pop

int launched(hipError_t e) { return e == hipSuccess && hipGetLastError() == hipSuccess ? 0 : kErr; }

}  // namespace

extern "C" {

// Each wrapper returns 0, or -1 for sizes outside what the probe reads
// safely or a failed launch.  `sink` holds 8 uint32 per workgroup.

int nvprobe_empty(int launches, hipStream_t s) {
    if (launches < 1) return kErr;
    for (int i = 0; i < launches; ++i) hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, s);
    return launched(hipSuccess);
}

// buf holds `bytes` bytes; bytes must equal workgroups * 256 * per_lane * 16.
int nvprobe_stream_read(const void* buf, int64_t bytes, int workgroups, int per_lane, uint32_t* sink,
                        uint64_t* clocks, hipStream_t s) {
    if (workgroups < 1 || bytes != int64_t(workgroups) * 256 * per_lane * 16) return kErr;
    const u32x4_t* b = static_cast<const u32x4_t*>(buf);
    switch (per_lane) {
        case 1: hipLaunchKernelGGL(stream_read_kernel<1>, dim3(workgroups), dim3(256), 0, s, b, sink, clocks); break;
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, dim3(workgroups), dim3(256), 0, s, b, sink, clocks); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3(workgroups), dim3(256), 0, s, b, sink, clocks); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3(workgroups), dim3(256), 0, s, b, sink, clocks); break;
        default: return kErr;
    }
    return launched(hipSuccess);
}

// iters must be a positive multiple of 8.
int nvprobe_lds_read(int workgroups, int iters, uint32_t* sink, uint64_t* clocks, hipStream_t s) {
    if (workgroups < 1 || iters < 8 || iters % 8) return kErr;
    hipLaunchKernelGGL(lds_read_kernel, dim3(workgroups), dim3(512), 0, s, iters, sink, clocks);
    return launched(hipSuccess);
}

// src holds `window` bytes, a positive multiple of 1024.  mode 0: copies to
// LDS (global_load_lds_dwordx4); 1: loads to registers; 2: loads to
// registers + ds_write_b128; 3: modes 0 and 2 in half the waves each.
// iters must be a positive multiple of inflight (8 or 16); reads (0 or 3)
// ds_read_b128 accompany each copy.  src and sink must be device pointers.
int nvprobe_copy(int mode, const void* src, int64_t window, int workgroups, int iters, int inflight, int reads,
                 uint32_t* sink, uint64_t* clocks, hipStream_t s) {
    if (src == nullptr || sink == nullptr) return kErr;
    if (workgroups < 1 || iters < 1 || window < 1024 || window % 1024) return kErr;
    if ((inflight != 8 && inflight != 16) || (reads != 0 && reads != 3)) return kErr;
    if (iters % inflight) return kErr;
    const char* p = static_cast<const char*>(src);
    const dim3 g(workgroups), b(512);
#define NVPROBE_COPY(F, R)                                                                              \
    if (mode == 0) hipLaunchKernelGGL((dma_kernel<F, R>), g, b, 0, s, p, window, iters, sink, clocks);   \
    else if (mode == 1) hipLaunchKernelGGL((vload_kernel<F, 0, R>), g, b, 0, s, p, window, iters, sink, clocks); \
    else if (mode == 2) hipLaunchKernelGGL((vload_kernel<F, 1, R>), g, b, 0, s, p, window, iters, sink, clocks); \
    else if (mode == 3) hipLaunchKernelGGL((hybrid_kernel<F, R>), g, b, 0, s, p, window, iters, sink, clocks);   \
    else return kErr;
    if (inflight == 8 && reads == 0) { NVPROBE_COPY(8, 0) }
    else if (inflight == 8) { NVPROBE_COPY(8, 3) }
    else if (reads == 0) { NVPROBE_COPY(16, 0) }
    else { NVPROBE_COPY(16, 3) }
#undef NVPROBE_COPY
    return launched(hipSuccess);
}

// dst holds tiles_m * 128 rows of `ld` bytes, ld >= tiles_n * 512.
int nvprobe_write_tiles(void* dst, int64_t ld, int tiles_m, int tiles_n, int nontemporal, uint64_t* clocks,
                        hipStream_t s) {
    if (tiles_m < 1 || tiles_n < 1 || ld < int64_t(tiles_n) * 512 || ld % 16) return kErr;
    char* d = static_cast<char*>(dst);
    if (nontemporal) hipLaunchKernelGGL(write_tiles_kernel<1>, dim3(tiles_m * tiles_n), dim3(512), 0, s, d, ld, tiles_n, clocks);
    else hipLaunchKernelGGL(write_tiles_kernel<0>, dim3(tiles_m * tiles_n), dim3(512), 0, s, d, ld, tiles_n, clocks);
    return launched(hipSuccess);
}

// 512-thread workgroups, `chains` independent accumulators per wave.
int nvprobe_mfma(int workgroups, int iters, int chains, uint32_t* sink, uint64_t* clocks, hipStream_t s) {
    if (workgroups < 1 || iters < 1) return kErr;
    if (chains == 4) hipLaunchKernelGGL(mfma_kernel<4>, dim3(workgroups), dim3(512), 0, s, iters, sink, clocks);
    else if (chains == 8) hipLaunchKernelGGL(mfma_kernel<8>, dim3(workgroups), dim3(512), 0, s, iters, sink, clocks);
    else return kErr;
    return launched(hipSuccess);
}

// The same with v_mfma_f32_16x16x32_bf16 (a quarter of the flops per
// instruction); chains 4, 8 or 16.
int nvprobe_mfma16(int workgroups, int iters, int chains, uint32_t* sink, uint64_t* clocks, hipStream_t s) {
    if (workgroups < 1 || iters < 1) return kErr;
    if (chains == 4) hipLaunchKernelGGL(mfma16_kernel<4>, dim3(workgroups), dim3(512), 0, s, iters, sink, clocks);
    else if (chains == 8) hipLaunchKernelGGL(mfma16_kernel<8>, dim3(workgroups), dim3(512), 0, s, iters, sink, clocks);
    else if (chains == 16) hipLaunchKernelGGL(mfma16_kernel<16>, dim3(workgroups), dim3(512), 0, s, iters, sink, clocks);
    else return kErr;
    return launched(hipSuccess);
}

// offsets: 64 byte offsets (host memory), each a multiple of width and at
// most 16384 - width; width 4, 8 or 16; write 0 (reads) or 1 (writes);
// iters a positive multiple of 8; cycles holds `workgroups` uint64.
int nvprobe_lds_map(const uint32_t* offsets, int width, int write, int workgroups, int iters, uint32_t* sink,
                    uint64_t* cycles, hipStream_t s) {
    if (offsets == nullptr || sink == nullptr || cycles == nullptr) return kErr;
    if (workgroups < 1 || iters < 8 || iters % 8 || (write != 0 && write != 1)) return kErr;
    if (width != 4 && width != 8 && width != 16) return kErr;
    LaneMap map;
    for (int l = 0; l < 64; ++l) {
        if (offsets[l] % uint32_t(width) || offsets[l] > uint32_t(16384 - width)) return kErr;
        map.off[l] = offsets[l];
    }
#define NVPROBE_LDS_MAP(W, WR) \
    hipLaunchKernelGGL((lds_map_kernel<W, WR>), dim3(workgroups), dim3(256), 0, s, map, iters, sink, cycles)
    if (write) {
        if (width == 16) NVPROBE_LDS_MAP(16, true);
        else if (width == 8) NVPROBE_LDS_MAP(8, true);
        else NVPROBE_LDS_MAP(4, true);
    } else {
        if (width == 16) NVPROBE_LDS_MAP(16, false);
        else if (width == 8) NVPROBE_LDS_MAP(8, false);
        else NVPROBE_LDS_MAP(4, false);
    }
#undef NVPROBE_LDS_MAP
    return launched(hipSuccess);
}

}  // extern "C"
