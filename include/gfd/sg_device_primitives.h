#pragma once
// GPU-side submission of scatter-gather lists, wave64 (HIP sources only).
// Same functions as the reference's include/gfd/sg_device_primitives.cuh:27-242
// (backpressure, entry / list allocation, commit, submit, completion waits);
// every function is wave-collective (all 64 lanes call it).
//
// MI355X differences: allocation counters are device-scope atomics on
// SGDeviceCounters in HBM (never atomics across PCIe into host memory);
// entries and headers are written to an SGTaskQueue (the host-resident one,
// or the session's HBM queue for a launch that sets
// SGDeviceCounters::dev_ring; the caller passes the one it posts to) with
// plain stores and committed with a system-scope release store of `sequence`;
// waits are bounded (a poll count, and the launch's deadline when it has one)
// and return false when they give up.
//
// Ring slots: list index i lives in lists[i % MAX_SG_LISTS].  Before the
// header of index i is written, the list that used the slot before it
// (i - MAX_SG_LISTS) must be done, i.e. the slot's `done` marker has reached
// i - MAX_SG_LISTS + 1.  This keeps the per-slot markers monotonic however
// the lists complete.
//
// A launch uses either host submitters (SGWarpSpecSession::submit_sg_list) or
// GPU submitters for its allocations, not both at once: the session seeds the
// device counters from the host counters when it launches.
#include "gfd/sg_task_queue.h"
#include "gfd/wave_ops.h"

namespace gfd {
namespace sg {

__device__ __forceinline__ SGDeviceCounters* counters(SGTaskQueue* sq) { return sg_device_counters(sq); }

__device__ __forceinline__ uint64_t atomic_add_dev(uint64_t* p, uint64_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_dev(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
// For polls: an agent-scope acquire invalidates the XCD's caches every time
// it runs, under every other wave on that XCD.  (With one wave polling this
// way through a 2 ms MoE launch, the three other workgroups on its XCD moved
// ~115 rows each; with relaxed polls ~155.)  The waits below poll with
// relaxed loads and make one acquire once their condition holds.
__device__ __forceinline__ uint64_t poll_dev(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The launch's deadline (SGDeviceCounters::deadline; 0: none), read once per
// wait, and whether it has passed.
__device__ __forceinline__ uint64_t launch_deadline(SGDeviceCounters* c) {
    return __hip_atomic_load(&c->deadline, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t launch_deadline(SGTaskQueue* sq) { return launch_deadline(counters(sq)); }
__device__ __forceinline__ bool past(uint64_t deadline) {
    return deadline != 0 && (uint64_t)wall_clock64() > deadline;
}

// Wait until `needed` more pool entries can be allocated without overwriting
// entries whose data has not landed yet.
__device__ __forceinline__ bool sg_wait_entry_space(SGTaskQueue* sq, uint32_t needed) {
    if (needed > (uint32_t)MAX_SG_POOL_ENTRIES) return false;
    SGDeviceCounters* c = counters(sq);
    const uint64_t dl = launch_deadline(sq);
    for (uint64_t n = 0; n < wave::kSpinLimit && !past(dl); n++) {
        const uint64_t alloc = poll_dev(&c->entry_alloc);
        const uint64_t done = poll_dev(&c->entries_done);
        if (alloc - done <= (uint64_t)(MAX_SG_POOL_ENTRIES - needed)) {
            wave::acquire_agent();
            return true;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// Wait until fewer than MAX_SG_LISTS - 1 lists of this launch are in flight.
__device__ __forceinline__ bool sg_wait_list_space(SGTaskQueue* sq) {
    SGDeviceCounters* c = counters(sq);
    const uint64_t dl = launch_deadline(sq);
    for (uint64_t n = 0; n < wave::kSpinLimit && !past(dl); n++) {
        const uint64_t in_flight = poll_dev(&c->list_alloc) - poll_dev(&c->list_base) - poll_dev(&c->lists_done);
        if (in_flight < (uint64_t)(MAX_SG_LISTS - 1)) {
            wave::acquire_agent();
            return true;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// Reserve `count` pool entries; returns the first pool index.
__device__ __forceinline__ uint64_t sg_alloc_entries(SGTaskQueue* sq, uint32_t count) {
    uint64_t base = 0;
    if (wave::lane_id() == 0) base = atomic_add_dev(&counters(sq)->entry_alloc, count);
    return wave::broadcast0(base);
}

// Copy `count` entries into the pool at pool_offset.
__device__ __forceinline__ void sg_write_entries(SGTaskQueue* sq, uint64_t pool_offset,
                                                 const DeviceSGEntry* src_entries, uint32_t count) {
    for (uint32_t i = (uint32_t)wave::lane_id(); i < count; i += wave::kWidth)
        sq->entries[(pool_offset + i) % MAX_SG_POOL_ENTRIES] = src_entries[i];
}

__device__ __forceinline__ void sg_write_entries_inline(SGTaskQueue* sq, uint64_t pool_offset,
                                                        const uint64_t* src_addrs, const uint64_t* dst_addrs,
                                                        const uint32_t* sizes, uint32_t tag, uint32_t count) {
    for (uint32_t i = (uint32_t)wave::lane_id(); i < count; i += wave::kWidth) {
        DeviceSGEntry& e = sq->entries[(pool_offset + i) % MAX_SG_POOL_ENTRIES];
        e.src_addr = src_addrs[i];
        e.dst_addr = dst_addrs[i];
        e.size = sizes[i];
        e.tag = tag;
    }
}

// Reserve one list ring index.
__device__ __forceinline__ uint64_t sg_alloc_list(SGTaskQueue* sq) {
    uint64_t slot = 0;
    if (wave::lane_id() == 0) slot = atomic_add_dev(&counters(sq)->list_alloc, 1);
    return wave::broadcast0(slot);
}

// Wait until ring index `slot` may be written: the list that held the ring
// slot before it is done.
__device__ __forceinline__ bool sg_wait_slot_free(SGTaskQueue* sq, uint64_t slot) {
    if (slot < (uint64_t)MAX_SG_LISTS) return true;
    const uint64_t want = slot - MAX_SG_LISTS + 1;
    const SGList& l = sq->lists[slot % MAX_SG_LISTS];
    const uint64_t dl = launch_deadline(sq);
    for (uint64_t n = 0; n < wave::kSpinLimit && !past(dl); n++) {
        if (__hip_atomic_load(const_cast<uint64_t*>(&l.done), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) >= want) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");  // system scope
            return true;
        }
        __builtin_amdgcn_s_sleep(32);
    }
    return false;
}

// Write the header and publish the list.  The system-scope release orders
// every entry and header store of this wave before the sequence store.
// False (nothing published) if the ring slot never became free.  slot_free:
// the caller knows the slot's previous list has landed (the session's
// gpu_lists_fit held for the launch), so the wait, a read of host memory, is
// skipped.
__device__ __forceinline__ bool sg_commit_list(SGTaskQueue* sq, uint64_t slot, uint32_t pool_offset,
                                               uint32_t count, uint32_t list_id, uint32_t flags,
                                               bool slot_free = false) {
    if (!slot_free && !sg_wait_slot_free(sq, slot)) {
        if (wave::lane_id() == 0)
            __hip_atomic_fetch_or(&counters(sq)->error, SG_ERR_RING_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    SGList& l = sq->lists[slot % MAX_SG_LISTS];
    if (wave::lane_id() == 0) {
        l.pool_offset = (uint32_t)(pool_offset % MAX_SG_POOL_ENTRIES);
        l.count = count;
        l.list_id = list_id;
        l.flags = flags;
        wave::store_system(&l.sequence, slot + 1);
    }
    return true;
}

// Backpressure + allocate + write + commit.  Returns the list ring index, or
// ~0 if a wait gave up.
__device__ __forceinline__ uint64_t sg_submit_list(SGTaskQueue* sq, const DeviceSGEntry* entries, uint32_t count,
                                                   uint32_t list_id, uint32_t flags = SG_FLAG_NONE) {
    if (!sg_wait_entry_space(sq, count) || !sg_wait_list_space(sq)) return ~0ull;
    const uint64_t pool_offset = sg_alloc_entries(sq, count);
    sg_write_entries(sq, pool_offset, entries, count);
    const uint64_t slot = sg_alloc_list(sq);
    if (!sg_commit_list(sq, slot, (uint32_t)(pool_offset % MAX_SG_POOL_ENTRIES), count, list_id, flags)) return ~0ull;
    return slot;
}

// Wait until at least `expected` lists have landed in HBM during this launch
// (host-submitted lists queued before it included, as the reference's
// lists_completed counts every list).
__device__ __forceinline__ bool sg_wait_list_done(SGTaskQueue* sq, uint64_t expected) {
    const uint64_t dl = launch_deadline(sq);
    for (uint64_t n = 0; n < wave::kSpinLimit && !past(dl); n++) {
        const uint64_t done = poll_dev(&counters(sq)->lists_done);
        if (done >= expected) {
            wave::acquire_agent();
            return true;
        }
        // Many lists still to land: a slower poll (~1 us) costs nothing.
        if (expected - done > 8) __builtin_amdgcn_s_sleep(32);
        else __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// Lists host submitters had queued when this launch started; they land
// during the launch and lists_done counts them.
__device__ __forceinline__ uint64_t sg_host_lists(SGTaskQueue* sq) {
    return __hip_atomic_load(&counters(sq)->host_lists, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until the `gpu_lists` lists this launch's GPU submitters post have
// landed, on top of the host lists queued before the launch.  Only then is
// every list of the launch known to have landed (the precondition of
// sg_terminate_all_landed).
__device__ __forceinline__ bool sg_wait_gpu_lists_done(SGTaskQueue* sq, uint64_t gpu_lists) {
    return sg_wait_list_done(sq, sg_host_lists(sq) + gpu_lists);
}

// Wait until list `list_id` has landed (d_list_done[list_id] != 0).
__device__ __forceinline__ bool sg_wait_list_id_done(SGTaskQueue* sq, uint32_t list_id) {
    if (list_id >= (uint32_t)MAX_SG_LISTS) return false;
    const uint64_t dl = launch_deadline(sq);
    for (uint64_t n = 0; n < wave::kSpinLimit && !past(dl); n++) {
        if (poll_dev(&sq->d_list_done[list_id]) != 0) {
            wave::acquire_agent();
            return true;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// Ask every transfer wave to exit once no committed list is left (a GPU
// submitter that has seen all its lists land calls this).
__device__ __forceinline__ void sg_terminate(SGTaskQueue* sq) {
    if (wave::lane_id() == 0)
        __hip_atomic_store(const_cast<uint32_t*>(&sq->terminate), 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// sg_terminate for a submitter whose sg_wait_list_done has just returned true
// for every list of the launch: with nothing left to copy, it also raises the
// HBM stop word that waiting transfer waves poll, so they exit without first
// having one of them read terminate across PCIe.  Not for any other case: a
// wave waiting for a committed list that no wave has seen yet would stop
// without copying it.
// c: the launch's counters, when the caller has their address (else they
// are found through the host queue, a read across PCIe).
__device__ __forceinline__ void sg_terminate_all_landed(SGTaskQueue* sq, SGDeviceCounters* c = nullptr) {
    sg_terminate(sq);
    if (wave::lane_id() == 0)
        __hip_atomic_store(&(c ? c : counters(sq))->stop, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// sg_wait_gpu_lists_done + sg_terminate_all_landed without a wave waiting:
// the transfer wave whose landing brings lists_done to host lists +
// gpu_lists ends the launch (SGDeviceCounters::stop_at).  Both sides are
// sequentially consistent (this wave stores stop_at, then reads lists_done;
// a lander adds to lists_done, then reads stop_at), so one of them sees the
// launch complete even when every list lands before stop_at is set.
// c as for sg_terminate_all_landed.
__device__ __forceinline__ void sg_stop_when_landed(SGTaskQueue* sq, uint64_t gpu_lists, SGDeviceCounters* c = nullptr) {
    if (!c) c = counters(sq);
    const uint64_t want = __hip_atomic_load(&c->host_lists, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + gpu_lists;
    int now = 0;
    if (wave::lane_id() == 0) {
        __hip_atomic_store(&c->stop_at, want, __ATOMIC_SEQ_CST, __HIP_MEMORY_SCOPE_AGENT);
        now = __hip_atomic_load(&c->lists_done, __ATOMIC_SEQ_CST, __HIP_MEMORY_SCOPE_AGENT) >= want;
    }
    if (__builtin_amdgcn_readfirstlane(now)) sg_terminate_all_landed(sq, c);
}

}  // namespace sg
}  // namespace gfd
