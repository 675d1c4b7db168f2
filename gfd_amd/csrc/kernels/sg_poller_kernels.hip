// The CPU poller's SG mode driven from a kernel: the reference's SG transfer
// warp protocol (include/gfd/sg_warp_spec.cuh:95-262) in which each list
// becomes descriptors with user_data = list_id << 32 | i and FLAG_LAST_IN_TILE
// on its last entry, the poller copies the list and raises d_list_done[id],
// and the workgroup then consumes the list.  SGWarpSpecSession kernels copy
// lists themselves; this path keeps the poller's process_batch_sg reachable
// from device code, and is what its GPU tests run.  Also the C-ABI that
// allocates an SGTaskQueue whose d_list_done the poller signals.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstring>

#include "gfd/device.h"
#include "gfd/sg_task_queue.h"
#include "gfd/tiled_queue.h"
#include "gfd_capi.h"

// Offsets the Python binding reads (gfd_amd.SGTaskQueue).
static_assert(offsetof(gfd::SGTaskQueue, list_alloc_idx) == 409600, "SGTaskQueue layout");
static_assert(offsetof(gfd::SGTaskQueue, lists_completed) == 409856, "SGTaskQueue layout");
static_assert(offsetof(gfd::SGTaskQueue, d_list_done) == 409872, "SGTaskQueue layout");

namespace {

// Workgroup l posts list l (entries [offs[l], offs[l+1]) of `entries`), waits
// (bounded) for its flag, then adds the u32-word checksum of every landed
// entry to sums[l].
__global__ __launch_bounds__(256) void sg_poller_kernel(gfd::DescriptorQueue* q, gfd::SGTaskQueue* sq,
                                                        const gfd::DeviceSGEntry* __restrict__ entries,
                                                        const uint32_t* __restrict__ offs, uint64_t max_ticks,
                                                        unsigned long long* __restrict__ sums, int* status) {
    __shared__ int ok;
    const uint32_t l = blockIdx.x;
    const uint32_t first = offs[l], count = offs[l + 1] - offs[l];
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63), nwaves = (int)(blockDim.x >> 6);
    if (threadIdx.x == 0) ok = 1;
    __syncthreads();
    if (wave == 0 && count > 0) {
        uint64_t base = 0;
        if (lane == 0)
            base = __hip_atomic_fetch_add(const_cast<uint64_t*>(&q->write_idx), (uint64_t)count, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_SYSTEM);
        base = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32)) << 32) |
               (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
        for (uint32_t i = (uint32_t)lane; i < count; i += 64) {
            const gfd::DeviceSGEntry e = entries[first + i];
            gfd::device::write_descriptor_raw(q, base + i, e.src_addr, e.dst_addr, e.size,
                                              i == count - 1 ? gfd::FLAG_LAST_IN_TILE : gfd::FLAG_NONE,
                                              ((uint64_t)l << 32) | i);
            gfd::device::commit_slot(q, base + i);
        }
        if (lane == 0) {
            const volatile uint64_t* flag = sq->d_list_done + l;
            const uint64_t t0 = wall_clock64();
            for (uint32_t n = 0;; n++) {
                if (gfd::device::load_relaxed_system(flag) != 0) break;  // every lane acquires below
                if (wall_clock64() - t0 > max_ticks) {
                    ok = 0;
                    break;
                }
                if (n >= 64) __builtin_amdgcn_s_sleep(8);
            }
        }
    }
    __syncthreads();
    if (!ok) {
        if (threadIdx.x == 0) __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return;
    }
    // The copy engines wrote the entries: every lane acquires before reading.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
    unsigned long long acc = 0;
    for (uint32_t i = (uint32_t)wave; i < count; i += (uint32_t)nwaves) {
        const gfd::DeviceSGEntry e = entries[first + i];
        const uint8_t* p = (const uint8_t*)e.dst_addr;
        const uint32_t nw = e.size / 4;
        if ((e.dst_addr & 3) == 0) {
            const uint32_t* w = (const uint32_t*)p;
            for (uint32_t k = (uint32_t)lane; k < nw; k += 64) acc += w[k];
        } else {
            for (uint32_t k = (uint32_t)lane; k < nw; k += 64)
                acc += (uint32_t)p[4 * k] | ((uint32_t)p[4 * k + 1] << 8) | ((uint32_t)p[4 * k + 2] << 16) |
                       ((uint32_t)p[4 * k + 3] << 24);
        }
        for (uint32_t b = nw * 4 + (uint32_t)lane; b < e.size; b += 64) acc += p[b];
    }
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)acc, o, 64);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(acc >> 32), o, 64);
        acc += ((unsigned long long)hi << 32) | lo;
    }
    if (lane == 0 && acc) atomicAdd(&sums[l], acc);
}

constexpr size_t kListWords = (size_t)gfd::MAX_SG_LISTS + gfd::SG_DEVICE_COUNTER_WORDS;
constexpr bool kSgPollerRunDisabled = true;

}  // namespace

extern "C" int gfd_sg_task_queue_alloc(void** out, int device_flags) {
    if (!out) return (int)hipErrorInvalidValue;
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, sizeof(gfd::SGTaskQueue), hipHostMallocCoherent);
    if (e != hipSuccess) return (int)e;
    std::memset(p, 0, sizeof(gfd::SGTaskQueue));
    void* d = nullptr;
    if (device_flags) {
        e = hipMalloc(&d, kListWords * sizeof(uint64_t));
        if (e == hipSuccess) e = hipMemset(d, 0, kListWords * sizeof(uint64_t));
        if (e == hipSuccess) e = hipDeviceSynchronize();
    } else {
        e = hipHostMalloc(&d, kListWords * sizeof(uint64_t), hipHostMallocCoherent);
        if (e == hipSuccess) std::memset(d, 0, kListWords * sizeof(uint64_t));
    }
    if (e != hipSuccess) {
        if (d) (void)(device_flags ? hipFree(d) : hipHostFree(d));
        (void)hipHostFree(p);
        return (int)e;
    }
    static_cast<gfd::SGTaskQueue*>(p)->d_list_done = static_cast<uint64_t*>(d);
    *out = p;
    return 0;
}

extern "C" int gfd_sg_task_queue_free(void* p) {
    if (!p) return 0;
    auto* sq = static_cast<gfd::SGTaskQueue*>(p);
    if (sq->d_list_done) {
        hipPointerAttribute_t a;
        const bool dev = hipPointerGetAttributes(&a, sq->d_list_done) == hipSuccess && a.type == hipMemoryTypeDevice;
        (void)hipGetLastError();
        (void)(dev ? hipFree(sq->d_list_done) : hipHostFree(sq->d_list_done));
    }
    return (int)hipHostFree(p);
}

extern "C" int gfd_sg_task_queue_reset(void* p) {
    if (!p) return (int)hipErrorInvalidValue;
    auto* sq = static_cast<gfd::SGTaskQueue*>(p);
    sq->lists_completed = 0;
    hipError_t e = hipMemset(sq->d_list_done, 0, kListWords * sizeof(uint64_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}

extern "C" int gfd_sg_poller_run(void* queue, void* sg_queue, const gfd_device_sg_entry* d_entries,
                                 const uint32_t* d_list_offsets, int num_lists, uint32_t total_entries,
                                 uint64_t timeout_us, unsigned long long* list_sums, int* status, void* stream) {
    if (!queue || !sg_queue || !d_entries || !d_list_offsets || !list_sums || !status || num_lists <= 0 ||
        num_lists > gfd::MAX_SG_LISTS)
        return (int)hipErrorInvalidValue;
    // Switched off: the first GPU run of this path (5 lists of 1 KiB entries,
    // lists split over batches, flags in HBM) aborted the process, and the
    // cause has not been found.  Nothing is launched until it is.
    if (kSgPollerRunDisabled) return (int)hipErrorNotSupported;
    auto* q = static_cast<gfd::DescriptorQueue*>(queue);
    auto* sq = static_cast<gfd::SGTaskQueue*>(sg_queue);
    if (!sq->d_list_done) return (int)hipErrorInvalidValue;
    // Slots are claimed without waiting for room: every list must fit the ring.
    const uint64_t used = q->write_idx - q->read_idx;
    if ((uint64_t)total_entries + used > (uint64_t)gfd::QUEUE_SIZE) return (int)hipErrorInvalidValue;
    const uint64_t ticks = timeout_us * (gfd::device::kWallClockHz / 1000000ull);
    hipLaunchKernelGGL(sg_poller_kernel, dim3((unsigned)num_lists), dim3(256), 0, (hipStream_t)stream, q, sq,
                       reinterpret_cast<const gfd::DeviceSGEntry*>(d_entries), d_list_offsets, ticks, list_sums,
                       status);
    return (int)hipGetLastError();
}
