#pragma once
// Scatter-gather task queue: per-list (src, dst, size) entries submitted by the
// host or by GPU waves, consumed by the SG transfer wave.  Same layout as
// include/gfd/sg_task_queue.h:28-88 of the reference (the queue lives in
// fine-grained host memory; d_list_done lives in HBM).
#include <cstdint>

namespace gfd {

constexpr int MAX_SG_LISTS = 512;
constexpr int MAX_SG_POOL_ENTRIES = 16384;

constexpr uint32_t SG_FLAG_NONE = 0;
constexpr uint32_t SG_FLAG_HOST_SUBMITTED = 1;

struct alignas(8) DeviceSGEntry {
    uint64_t src_addr;
    uint64_t dst_addr;
    uint32_t size;
    uint32_t tag;
};
static_assert(sizeof(DeviceSGEntry) == 24, "DeviceSGEntry must be 24 bytes");

struct alignas(16) SGList {
    uint32_t pool_offset;        // first entry in the pool (mod MAX_SG_POOL_ENTRIES)
    uint32_t count;
    uint32_t list_id;
    uint32_t flags;
    volatile uint64_t sequence;  // ring slot + 1 when committed
    uint64_t _pad;
};
static_assert(sizeof(SGList) == 32, "SGList must be 32 bytes");

struct SGTaskQueue {
    SGList lists[MAX_SG_LISTS];
    DeviceSGEntry entries[MAX_SG_POOL_ENTRIES];

    alignas(64) volatile uint64_t list_alloc_idx;
    alignas(64) volatile uint64_t entry_alloc_idx;

    alignas(64) volatile uint64_t list_read_idx;
    alignas(64) volatile uint64_t entry_consumed_idx;

    alignas(64) volatile uint64_t lists_completed;
    volatile uint32_t terminate;
    uint32_t _pad_term;

    uint64_t* d_list_done;  // HBM, one u64 per list id
};

namespace sg_compat {

// Linear mapping -> SG entries: entry i copies token (start_idx + i) from
// cpu_base + idx*token_size to gpu_base + idx*token_size
// (include/gfd/sg_task_queue.h:106-122 of the reference).
inline void linear_to_sg_entries(DeviceSGEntry* entries, const void* cpu_base, void* gpu_base,
                                 uint32_t token_size, uint32_t start_idx, uint32_t count,
                                 uint32_t tag = 0) {
    for (uint32_t i = 0; i < count; i++) {
        const uint64_t idx = (uint64_t)start_idx + i;
        entries[i].src_addr = (uint64_t)(uintptr_t)cpu_base + idx * token_size;
        entries[i].dst_addr = (uint64_t)(uintptr_t)gpu_base + idx * token_size;
        entries[i].size = token_size;
        entries[i].tag = tag;
    }
}

}  // namespace sg_compat
}  // namespace gfd
