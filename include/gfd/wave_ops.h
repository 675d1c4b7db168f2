#pragma once
// Wave64 building blocks shared by the gfx950 kernels (HIP sources only):
// whole-wave copies of host->HBM byte ranges, lane broadcasts, bounded LDS
// waits with s_sleep back-off, and the fences of the producer/consumer
// hand-off.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace gfd {
namespace wave {

constexpr int kWidth = 64;
// Polls of an LDS / memory flag before a wait gives up (~1-2 s with s_sleep 1).
constexpr uint64_t kSpinLimit = 1ull << 26;

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWidth - 1)); }
__device__ __forceinline__ int wave_id() { return (int)(threadIdx.x / kWidth); }

__device__ __forceinline__ uint64_t readlane64(uint64_t x, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t broadcast0(uint64_t x) { return readlane64(x, 0); }

// Copy n bytes s -> d with the whole wave: 16-byte vectors (U in flight per
// lane) when d and s share their alignment mod 16, bytes otherwise.
template <int U = 4>
__device__ __forceinline__ void copy(uint64_t d, uint64_t s, uint64_t n) {
    const uint32_t lane = (uint32_t)lane_id();
    if (((d ^ s) & 15) == 0) {
        uint64_t head = (16 - (d & 15)) & 15;
        if (head > n) head = n;
        if (lane < head) *reinterpret_cast<uint8_t*>(d + lane) = *reinterpret_cast<const uint8_t*>(s + lane);
        d += head;
        s += head;
        n -= head;
        const uint64_t nv = n >> 4;
        const uint4* sv = reinterpret_cast<const uint4*>(s);
        uint4* dv = reinterpret_cast<uint4*>(d);
        for (uint64_t base = 0; base < nv; base += (uint64_t)kWidth * U) {
            uint4 r[U];
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint64_t v = base + (uint64_t)k * kWidth + lane;
                if (v < nv) r[k] = sv[v];
            }
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint64_t v = base + (uint64_t)k * kWidth + lane;
                if (v < nv) dv[v] = r[k];
            }
        }
        const uint64_t tail = n & 15;
        if (lane < tail)
            *reinterpret_cast<uint8_t*>(d + (nv << 4) + lane) = *reinterpret_cast<const uint8_t*>(s + (nv << 4) + lane);
    } else {
        for (uint64_t b = lane; b < n; b += kWidth)
            *reinterpret_cast<uint8_t*>(d + b) = *reinterpret_cast<const uint8_t*>(s + b);
    }
}

// Make this wave's global stores visible device-wide before a flag is raised
// (producer side) / see other waves' stores after a flag is seen (consumer).
__device__ __forceinline__ void release_agent() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ __forceinline__ void acquire_agent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

__device__ __forceinline__ int lds_load(const int* p) {
    return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(int* p, int v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Bounded waits: true once the condition holds, false after kSpinLimit polls.
__device__ __forceinline__ bool wait_lds_eq(const int* p, int want) {
    for (uint64_t n = 0; n < kSpinLimit; n++) {
        if (lds_load(p) == want) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}
__device__ __forceinline__ bool wait_lds_gt(const int* p, int than) {
    for (uint64_t n = 0; n < kSpinLimit; n++) {
        if (lds_load(p) > than) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}
__device__ __forceinline__ bool wait_lds_ne(const int* p, int old) {
    for (uint64_t n = 0; n < kSpinLimit; n++) {
        if (lds_load(p) != old) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

__device__ __forceinline__ uint64_t load_system(const volatile uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_system(volatile uint64_t* p, uint64_t v) {
    __hip_atomic_store(const_cast<uint64_t*>(p), v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t load_system32(const volatile uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace wave
}  // namespace gfd
