// Memory-system probe used by bench.py to price the on-chip roof of the SpMM
// kernels (not part of the SpMM/SDDMM boundary; built as libbsp_probe.so).
//
// bsp_probe_dma_stream: `grid` workgroups of `waves` waves; each wave streams
// `iters` loads of 1 KB (global_load_lds_dwordx4, the SpMM kernels' load path)
// from a buffer into a wave-private LDS ring, at most 16 in flight.  Wave w of
// workgroup g starts at a hashed 1 KB-aligned offset and steps by 997 KB, both
// taken modulo `region_bytes` (a power of two): a 2 MB region stays resident
// in every XCD's L2, a large one streams from HBM.  Every address is inside
// the region and every LDS write inside the workgroup's allocation.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | (((N >> 4) & 0x3) << 14));
    __asm__ volatile("" ::: "memory");
}

__global__ __launch_bounds__(1024) void dma_stream(const uint8_t* src, uint64_t mask, int iters) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t ring[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t gw = (uint64_t)blockIdx.x * (blockDim.x >> 6) + wave;
    uint64_t off = (gw * 0x9E3779B97F4A7C15ull) & mask & ~1023ull;
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring + wave * 8192;
    for (int i = 0; i < iters; ++i) {
        const void* g = src + ((off + lane * 16) & mask);
        const uint32_t lds = __builtin_amdgcn_readfirstlane(base + (i & 7) * 1024);
        __asm__ volatile(
            "s_mov_b32 m0, %1\n\t"
            "global_load_lds_dwordx4 %0, off"
            :
            : "v"(g), "s"(lds)
            : "memory");
        off = (off + 1024 * 997) & mask;
        wait_vmcnt<16>();
    }
    wait_vmcnt<0>();
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" {

// region_bytes: a power of two >= 1 KB, buf at least that long (16-byte aligned);
// waves 1..16; 8 KB of LDS per wave.  Returns a hipError_t.
int bsp_probe_dma_stream(const void* buf, int64_t region_bytes, int grid, int waves, int iters, void* stream) {
    if (!buf || region_bytes < 1024 || (region_bytes & (region_bytes - 1)) || grid <= 0 || waves < 1 ||
        waves > 16 || iters <= 0)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(dma_stream, dim3(grid), dim3(64 * waves), (size_t)waves * 8192, (hipStream_t)stream,
                       (const uint8_t*)buf, (uint64_t)(region_bytes - 1), iters);
    return (int)hipGetLastError();
}

// An empty kernel of `grid` workgroups (the fixed cost of a launch).
int bsp_probe_empty(int grid, void* stream) {
    if (grid <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream);
    return (int)hipGetLastError();
}

}  // extern "C"
