#pragma once
// Scatter-gather task queue: per-list (src, dst, size) entries submitted by the
// host or by GPU waves, consumed by the SG transfer wave.  Same layout as
// include/gfd/sg_task_queue.h:28-88 of the reference (the queue lives in
// fine-grained host memory; d_list_done lives in HBM).
#include <cstdint>

#ifdef __HIPCC__
#define GFD_HD __host__ __device__
#else
#define GFD_HD
#endif

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
    volatile uint64_t sequence;  // ring slot + 1 when committed, 0 once claimed
    // The reference's padding word.  Here it holds "ring index + 1" once the
    // list's data has landed in HBM: a completion marker the host polls
    // without reading device memory.  A ring slot is refilled only after the
    // previous list in it is done, so per slot this value only grows.
    volatile uint64_t done;
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
    // The reference's padding word after `terminate`.  This library reads it as
    // the transfer waves' idle limit in milliseconds (0 = 30 s): a wave that
    // sees no committed list for that long gives up instead of spinning
    // forever when the host never sets `terminate`.
    uint32_t idle_limit_ms;

    uint64_t* d_list_done;  // HBM, one u64 per list id (+ SGDeviceCounters after them)
};

// Claim / allocation counters kept in HBM right after d_list_done[MAX_SG_LISTS]
// (sessions allocate MAX_SG_LISTS + SG_DEVICE_COUNTER_WORDS words).  GPU waves
// update them with device-scope atomics, so no atomic operation ever crosses
// PCIe into host memory.
struct SGDeviceCounters {
    uint64_t list_claim;      // next ring index a transfer wave claims
    uint64_t list_alloc;      // next ring index a GPU submitter allocates
    uint64_t entry_alloc;     // next pool index a GPU submitter allocates
    // Entries landed, counted on from the first pool index of the launch, so
    // entry_alloc - entries_done is the pool occupancy (exact while lists land
    // in submission order, as the reference's entry_consumed_idx).
    uint64_t entries_done;
    uint64_t lists_done;      // lists landed during this launch
    uint64_t error;           // nonzero: a bounded wait gave up (bit flags)
    // Lowest ring index whose commit no transfer wave has seen yet.  Only the
    // wave holding this index polls host memory; the others poll this word.
    uint64_t list_known;
    uint64_t stop;            // set once `terminate` has been seen: waiting waves exit
    uint64_t list_base;       // first ring index of this launch
    uint64_t bytes_done;      // bytes landed during this launch
    uint64_t helpers;         // transfer helper waves per workgroup (waves 2 .. 1 + helpers)
    // Compute waves per workgroup that share each landed list (waves 1 ..
    // compute_waves), for compute functors that declare kSharesLists; 0 or 1
    // and every other functor: wave 1 alone.
    uint64_t compute_waves;
    // Per-list timeline (0: off).  Device address of trace_cap SGTraceList
    // records, one per ring index of the launch (list_base + k -> record k),
    // followed by trace_blocks SGTraceBlock records, one per workgroup.
    uint64_t trace;
    uint64_t trace_cap;
    uint64_t trace_blocks;
    // Lists host submitters had queued before this launch.  They land during
    // it, so lists_done counts them: a GPU submitter waiting for its own
    // `total` lists waits for lists_done >= host_lists + total.
    uint64_t host_lists;
    // Launch-wide deadline on the GPU's 100 MHz wall clock (wall_clock64()),
    // or 0 for none.  Launches whose lists all come from GPU submitters set
    // it: every wait of the launch (transfer, helper and compute waves, and
    // the sg:: submitter waits) gives up once it has passed, so a protocol
    // stall ends the kernel with an error bit instead of spinning.
    uint64_t deadline;
    // Device address of an SGTaskQueue in HBM (0: none) holding the lists
    // that this launch's GPU submitters post: ring indices from list_base +
    // host_lists on.  Their headers and entries are then written and read in
    // HBM, never across PCIe; the header's `done` marker is still raised in
    // the host queue too, where host code and host submitters look for it.
    uint64_t dev_ring;
    // Pool index of this launch's first GPU-submitted entry (entry_alloc as
    // the launch starts), for submitters that place their lists at fixed
    // positions instead of allocating them.
    uint64_t entry_first;
    // lists_done at which the transfer wave that lands that list ends the
    // launch (terminate + stop), as sg_terminate_all_landed would; 0: off.
    // Set by a GPU submitter with sg_stop_when_landed.
    uint64_t stop_at;
    // The transfer and compute waves' idle limit in 100 MHz wall-clock ticks
    // (SGTaskQueue::idle_limit_ms, 0 meaning 30 s, as the launch starts), so
    // they need not read it from the host queue across PCIe; 0: not set,
    // read it there.
    uint64_t idle_ticks;
    uint64_t _pad[3];
};

// One list of a traced launch, in wall-clock ticks (100 MHz): when its
// transfer wave started looking for it, when its header had been read (the
// copy starts), and when its bytes had been released device-wide.  Records of
// ring indices beyond trace_cap are not written; a record still 0 was not
// claimed.
struct SGTraceList {
    uint64_t claimed;
    uint64_t ready;
    uint64_t landed;
    uint32_t block;
    uint32_t list_id;
};
static_assert(sizeof(SGTraceList) == 32, "SGTraceList must be 32 bytes");

// One workgroup of a traced launch: when its transfer wave started and
// exited, and how many lists it copied.
struct SGTraceBlock {
    uint64_t start;
    uint64_t exit;
    uint64_t lists;
    // Where the workgroup ran: XCC_ID << 32 | HW_ID of its transfer wave
    // (HW_ID: CU id in bits 8-11, shader array 12, shader engine 13-15).
    uint64_t hw;
};
static_assert(sizeof(SGTraceBlock) == 32, "SGTraceBlock must be 32 bytes");
constexpr int SG_DEVICE_COUNTER_WORDS = (int)(sizeof(SGDeviceCounters) / sizeof(uint64_t));

// Bits of SGDeviceCounters::error.
constexpr uint64_t SG_ERR_SLOT_WAIT = 1;     // transfer wave: the compute wave never freed an LDS slot
constexpr uint64_t SG_ERR_COMPUTE_WAIT = 2;  // compute wave: the transfer wave never handed a list over
constexpr uint64_t SG_ERR_RING_WAIT = 4;     // GPU submitter: a ring slot never became free
constexpr uint64_t SG_ERR_HELPER_WAIT = 8;   // transfer waves: a copy job's hand-off stalled
constexpr uint64_t SG_ERR_BAD_ROW = 16;      // GPU submitter: a routing entry out of range (skipped)
constexpr uint64_t SG_ERR_LIST_WAIT = 32;    // GPU submitter: its lists did not all land in time
constexpr uint64_t SG_ERR_DEADLINE = 64;     // transfer wave: gave up at the launch's deadline
static_assert(sizeof(SGDeviceCounters) == 192, "SGDeviceCounters is three cache lines");

GFD_HD inline SGDeviceCounters* sg_device_counters(const SGTaskQueue* sq) {
    return reinterpret_cast<SGDeviceCounters*>(sq->d_list_done + MAX_SG_LISTS);
}

// The d_list_done array the counters follow (device code given the counters'
// address needs no read of the host queue to find it).
GFD_HD inline uint64_t* sg_list_done_words(SGDeviceCounters* c) {
    return reinterpret_cast<uint64_t*>(c) - MAX_SG_LISTS;
}

// SGDeviceCounters::idle_ticks for an idle limit in ms (0 meaning 30 s).
GFD_HD inline uint64_t sg_idle_ticks(uint32_t idle_limit_ms) {
    return (uint64_t)(idle_limit_ms ? idle_limit_ms : 30000u) * 100000ull;
}

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
