// Host-side launch helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <unordered_map>

#define TCQ_MAX_WIDTH 16384

// Kernels that need more than 64 KiB of dynamic LDS (gfx950 holds 160 KiB per workgroup, static + dynamic) opt in to the
// size they ask for; the largest size granted so far is remembered per kernel.
static inline void allow_lds(const void* fn, size_t bytes) {
    static std::mutex mu;
    static std::unordered_map<const void*, size_t> granted;
    if (bytes <= 65536) return;
    std::lock_guard<std::mutex> lock(mu);
    auto it = granted.find(fn);
    if (it != granted.end() && it->second >= bytes) return;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess) granted[fn] = bytes;
}

template <typename... KArgs, typename... Args>
static inline void launch_k(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem, hipStream_t stream, Args... args) {
    (void)hipGetLastError();  // the status returned below belongs to this launch only
    allow_lds((const void*)kernel, shmem);
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, static_cast<KArgs>(args)...);
}

static inline int launch_status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}
