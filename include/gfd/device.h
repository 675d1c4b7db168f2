#pragma once
// Device-side descriptor API for wave64 HIP kernels on gfx950
// (the reference's include/gfd/device.cuh:46-175: write_descriptor,
// fence_and_commit, write_and_commit, wait_for_completion,
// write_descriptor_safe).  Include from HIP sources only.
//
// Ordering on MI355X: descriptor bodies are two 16-byte stores into
// fine-grained host memory; the commit is a system-scope release store of
// `sequence = slot + 1`.  One wave executes the release once for all 64 lanes,
// so no leader-lane fence dance is needed.  Waits poll done_idx with
// system-scope acquire loads and s_sleep back-off, and are bounded.
#include <hip/hip_runtime.h>

#include "gfd/descriptor_queue.h"

namespace gfd {
namespace device {

// s_memrealtime ticks at 100 MHz on gfx9 parts (MI300/MI355X).
constexpr uint64_t kWallClockHz = 100000000ull;
constexpr uint64_t kDefaultWaitTicks = 10ull * kWallClockHz;  // 10 s

__device__ __forceinline__ uint64_t load_acquire_system(const volatile uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}
// Polls read with relaxed loads and make one acquire (fence) once their
// condition holds: an acquire invalidates the caches of the wave's XCD every
// time it runs, which slows every other wave there.
__device__ __forceinline__ uint64_t load_relaxed_system(const volatile uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void acquire_system() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, ""); }

__device__ __forceinline__ void store_release_system(volatile uint64_t* p, uint64_t v) {
    __hip_atomic_store(const_cast<uint64_t*>(p), v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Descriptor for token `token_idx` at slot base_slot + token_idx: dst =
// gpu_dst + token_idx * token_size, LAST_IN_BATCH on token num_tokens-1.
__device__ __forceinline__ void write_descriptor(DescriptorQueue* queue, uint64_t base_slot, int token_idx,
                                                 uint64_t src_addr, void* gpu_dst, uint32_t token_size,
                                                 int num_tokens, uint64_t user_data = 0) {
    const uint64_t slot = base_slot + (uint64_t)token_idx;
    Descriptor* d = &queue->entries[slot % QUEUE_SIZE];
    const uint64_t dst = (uint64_t)(uintptr_t)gpu_dst + (uint64_t)token_idx * token_size;
    const uint32_t flags = (token_idx == num_tokens - 1) ? FLAG_LAST_IN_BATCH : FLAG_NONE;
    ulonglong2* body = reinterpret_cast<ulonglong2*>(d);
    body[0] = make_ulonglong2(src_addr, dst);
    body[1] = make_ulonglong2(((uint64_t)flags << 32) | token_size, user_data);
}

// Descriptor with explicit fields (SG / tiled transfer waves).
__device__ __forceinline__ void write_descriptor_raw(DescriptorQueue* queue, uint64_t slot, uint64_t src_addr,
                                                     uint64_t dst_addr, uint32_t size, uint32_t flags,
                                                     uint64_t user_data) {
    Descriptor* d = &queue->entries[slot % QUEUE_SIZE];
    ulonglong2* body = reinterpret_cast<ulonglong2*>(d);
    body[0] = make_ulonglong2(src_addr, dst_addr);
    body[1] = make_ulonglong2(((uint64_t)flags << 32) | size, user_data);
}

__device__ __forceinline__ void commit_slot(DescriptorQueue* queue, uint64_t slot) {
    store_release_system(&queue->entries[slot % QUEUE_SIZE].sequence, slot + 1);
}

// Publish this lane's descriptor (if active) to the CPU poller.
__device__ __forceinline__ void fence_and_commit(DescriptorQueue* queue, uint64_t base_slot, int token_idx,
                                                 bool active) {
    if (active) commit_slot(queue, base_slot + (uint64_t)token_idx);
}

__device__ __forceinline__ void write_and_commit(DescriptorQueue* queue, uint64_t base_slot, int token_idx,
                                                 bool active, uint64_t src_addr, void* gpu_dst,
                                                 uint32_t token_size, int num_tokens, uint64_t user_data = 0) {
    if (active) {
        write_descriptor(queue, base_slot, token_idx, src_addr, gpu_dst, token_size, num_tokens, user_data);
        commit_slot(queue, base_slot + (uint64_t)token_idx);
    }
}

// Write only if the ring has room at this slot; false if it is full there (the
// caller retries).  Room means the slot's previous use, slot - QUEUE_SIZE, has
// been consumed: the poller's read_idx has passed it (the poller zeroes a
// slot's sequence before it publishes read_idx past the slot).  The reference
// tests sequence == 0 instead (device.cuh:129-152), which cannot tell a
// consumed slot from one whose previous use has not been written yet: when
// one launch spans more than QUEUE_SIZE slots, a writer of the later lap can
// run first, overwrite the slot, and the poller then waits forever for the
// earlier descriptor.
__device__ __forceinline__ bool write_descriptor_safe(DescriptorQueue* queue, uint64_t base_slot, int token_idx,
                                                      uint64_t src_addr, void* gpu_dst, uint32_t token_size,
                                                      int num_tokens, uint64_t user_data = 0) {
    const uint64_t slot = base_slot + (uint64_t)token_idx;
    if (slot >= (uint64_t)QUEUE_SIZE) {
        if (load_relaxed_system(&queue->read_idx) <= slot - (uint64_t)QUEUE_SIZE) return false;
        acquire_system();  // the slot's consumption before this lane's writes
    }
    write_descriptor(queue, base_slot, token_idx, src_addr, gpu_dst, token_size, num_tokens, user_data);
    return true;
}

// Spin (one lane) until done_idx >= expected_done or `max_ticks` of the
// 100 MHz wall clock pass.  Returns true on completion.
__device__ __forceinline__ bool wait_for_completion(DescriptorQueue* queue, uint64_t expected_done,
                                                    uint64_t max_ticks = kDefaultWaitTicks) {
    const uint64_t t0 = wall_clock64();
    for (;;) {
        if (load_relaxed_system(&queue->done_idx) >= expected_done) {
            acquire_system();
            return true;
        }
        if (wall_clock64() - t0 > max_ticks) return false;
        __builtin_amdgcn_s_sleep(4);
    }
}

}  // namespace device
}  // namespace gfd
