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

// 16-byte vector as a native clang vector: arrays of these stay in VGPRs at
// any unroll (arrays of HIP's uint4 wrapper go to scratch from 8 on).
typedef uint32_t vec4u __attribute__((ext_vector_type(4)));
// Global-address-space views, so copies compile to global_load/global_store
// (flat instructions would also wait on the LDS counter).
typedef __attribute__((address_space(1))) vec4u gvec4u;

__device__ __forceinline__ vec4u gload(uint64_t a) { return *reinterpret_cast<const gvec4u*>(a); }
__device__ __forceinline__ void gstore(uint64_t a, vec4u v) { *reinterpret_cast<gvec4u*>(a) = v; }

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
        // Branch-free: a lane past the end works on the last vector instead
        // (loads it and stores the same bytes back).  A guarded load or store
        // sits in its own basic block, and the compiler then waits for every
        // earlier memory operation first, which leaves one in flight.
        for (uint64_t base = 0; base < nv; base += (uint64_t)kWidth * U) {
            vec4u r[U];
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint64_t v = base + (uint64_t)k * kWidth + lane;
                r[k] = gload(s + ((v < nv ? v : nv - 1) << 4));
            }
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint64_t v = base + (uint64_t)k * kWidth + lane;
                gstore(d + ((v < nv ? v : nv - 1) << 4), r[k]);
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

// 16-byte loads in flight per lane of a transfer wave, from the number of
// transfer waves in the grid: about 1 MiB of host reads outstanding in total
// (64 lanes x U x 16 B per wave) fills the PCIe link; far more only queues
// (measured on MI355X: 8 waves reach 48 GB/s at U = 16 but 20 GB/s at
// U = 4, while 256 waves drop from 55 to 47 GB/s at U = 16).
__device__ __forceinline__ int transfer_unroll(uint32_t transfer_waves) {
    return transfer_waves <= 64 ? 16 : (transfer_waves <= 128 ? 8 : 4);
}

template <int U>
__device__ __forceinline__ void copy(uint64_t d, uint64_t s, uint64_t n);

// copy() with U chosen at run time (16, 8 or 4).
__device__ __forceinline__ void copy_u(int u, uint64_t d, uint64_t s, uint64_t n) {
    if (u >= 16) copy<16>(d, s, n);
    else if (u >= 8) copy<8>(d, s, n);
    else copy<4>(d, s, n);
}

// Per-wave LDS scratch for copy_batch: start vector and addresses of up to 64 entries.
struct BatchLds {
    uint32_t start[kWidth + 1];
    uint64_t src[kWidth];
    uint64_t dst[kWidth];
};

// The flat vector stream of copy_batch: vector v of the batch belongs to entry
// e (v / vpe when every entry has vpe vectors, else the last entry whose
// start is <= v, found by a fixed 6-step search) at offset v - start[e].
template <int U, bool kUniform>
__device__ __forceinline__ void flat_copy(uint32_t total, uint32_t vpe, uint32_t nb, const BatchLds* lds) {
    const uint32_t lane = (uint32_t)lane_id();
    for (uint32_t base = 0; base < total; base += (uint32_t)kWidth * U) {
        vec4u r[U];
        uint64_t da[U];
#pragma unroll
        for (int k = 0; k < U; k++) {
            // Branch-free on a clamped index, as in copy().
            const uint32_t v0 = base + (uint32_t)k * kWidth + lane;
            const uint32_t v = v0 < total ? v0 : total - 1;
            uint32_t e, o;
            if (kUniform) {
                e = v / vpe;
                o = v - e * vpe;
            } else {
                e = 0;
#pragma unroll
                for (uint32_t step = kWidth / 2; step > 0; step >>= 1)
                    if (e + step < nb && lds->start[e + step] <= v) e += step;
                o = v - lds->start[e];
            }
            r[k] = gload(lds->src[e] + ((uint64_t)o << 4));
            da[k] = lds->dst[e] + ((uint64_t)o << 4);
        }
#pragma unroll
        for (int k = 0; k < U; k++) gstore(da[k], r[k]);
    }
}

// flat_copy() staged through LDS: each lane's 16 bytes go host -> LDS with
// global_load_lds_dwordx4 (no VGPRs held while the loads are in flight), then
// LDS -> VGPR -> HBM.  `stage` is this wave's LDS area of U * 64 vectors.
typedef __attribute__((address_space(1))) const void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

template <int U, bool kUniform>
__device__ __forceinline__ void flat_copy_lds(uint32_t total, uint32_t vpe, uint32_t nb, const BatchLds* lds,
                                              vec4u* stage) {
    const uint32_t lane = (uint32_t)lane_id();
    for (uint32_t base = 0; base < total; base += (uint32_t)kWidth * U) {
        uint64_t da[U];
#pragma unroll
        for (int k = 0; k < U; k++) {
            const uint32_t v0 = base + (uint32_t)k * kWidth + lane;
            const uint32_t v = v0 < total ? v0 : total - 1;
            uint32_t e, o;
            if (kUniform) {
                e = v / vpe;
                o = v - e * vpe;
            } else {
                e = 0;
#pragma unroll
                for (uint32_t step = kWidth / 2; step > 0; step >>= 1)
                    if (e + step < nb && lds->start[e + step] <= v) e += step;
                o = v - lds->start[e];
            }
            // lane l's 16 bytes land at stage[k * 64 + l]
            __builtin_amdgcn_global_load_lds((gptr_t)(uintptr_t)(lds->src[e] + ((uint64_t)o << 4)),
                                             (lptr_t)(stage + k * kWidth), 16, 0, 0);
            da[k] = lds->dst[e] + ((uint64_t)o << 4);
        }
        __builtin_amdgcn_s_waitcnt(0);  // every load has landed in LDS
#pragma unroll
        for (int k = 0; k < U; k++) gstore(da[k], stage[k * kWidth + lane]);
    }
}

// Copy a batch of nb <= 64 entries, lane j holding entry j's (dst, src, bytes).
// When every entry is 16-byte aligned on both sides with a size that is a
// multiple of 16, the batch is copied as one stream of 16-byte vectors across
// entry boundaries: u loads in flight per lane when all entries have the same
// size (u = 16, 8 or 4), 4 otherwise.  Other batches go entry by entry.
// Returns the bytes copied.
__device__ __forceinline__ uint64_t copy_batch(int u, uint64_t md, uint64_t ms, uint64_t mn, uint32_t nb,
                                               BatchLds* lds, vec4u* stage = nullptr) {
    const uint32_t lane = (uint32_t)lane_id();
    const bool mine = lane < nb;
    const bool aligned = !mine || (((md | ms | mn) & 15) == 0 && (mn >> 4) < (1ull << 26));
    uint64_t total_bytes = 0;
    for (uint32_t j = 0; j < nb; j++) total_bytes += readlane64(mn, (int)j);
    if (__ballot(!aligned) != 0) {
        for (uint32_t j = 0; j < nb; j++) copy<4>(readlane64(md, (int)j), readlane64(ms, (int)j), readlane64(mn, (int)j));
        return total_bytes;
    }
    // 64 entries of < 2^26 vectors each: the batch's vector index fits 32 bits.
    const uint32_t vecs = mine ? (uint32_t)(mn >> 4) : 0u;
    uint32_t incl = vecs;
#pragma unroll
    for (int o = 1; o < kWidth; o <<= 1) {
        const uint32_t t = (uint32_t)__shfl_up((int)incl, o, kWidth);
        if (lane >= (uint32_t)o) incl += t;
    }
    if (mine) {
        lds->start[lane] = incl - vecs;
        lds->src[lane] = ms;
        lds->dst[lane] = md;
    }
    const uint32_t total = (uint32_t)(total_bytes >> 4);
    if (lane == 0) lds->start[nb] = total;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t vpe0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)vecs);
    if (total > 0) {
        const bool uniform = __ballot(mine && vecs != vpe0) == 0;
        if (stage) {  // LDS-staged, `u` vectors per lane (the caller sized stage for it)
            if (!uniform) flat_copy_lds<4, false>(total, 0, nb, lds, stage);
            else if (u >= 16) flat_copy_lds<16, true>(total, vpe0, nb, lds, stage);
            else if (u >= 8) flat_copy_lds<8, true>(total, vpe0, nb, lds, stage);
            else flat_copy_lds<4, true>(total, vpe0, nb, lds, stage);
        } else if (uniform) {
            if (u >= 16) flat_copy<16, true>(total, vpe0, nb, lds);
            else if (u >= 8) flat_copy<8, true>(total, vpe0, nb, lds);
            else flat_copy<4, true>(total, vpe0, nb, lds);
        } else {
            flat_copy<4, false>(total, 0, nb, lds);
        }
    }
    __builtin_amdgcn_wave_barrier();  // lds reused by the next batch
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    return total_bytes;
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

// Completion of a whole grid signalled to the host without a stream
// synchronisation.  Every wave of the grid calls it once after its last
// store: the wave releases its stores at agent scope and counts itself in
// `counter` (HBM, 0 before the launch); the last wave of `total_waves`
// acquires them, puts the counter back to 0 for the next launch, and stores
// `value` to `host_word` (pinned host memory) with a system-scope release, so
// every byte the grid wrote is visible to any agent once the host reads
// `value` there.  A null host_word disables it.
struct GridDone {
    unsigned int* counter;
    uint64_t* host_word;
    uint64_t value;
};

__device__ __forceinline__ void signal_grid_done(const GridDone& g, uint32_t total_waves) {
    if (!g.host_word) return;
    release_agent();
    if (lane_id() == 0) {
        const unsigned int prev = __hip_atomic_fetch_add(g.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (prev + 1 == total_waves) {
            __hip_atomic_store(g.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(g.host_word, g.value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

}  // namespace wave
}  // namespace gfd
