#pragma once
// GPU -> CPU request ring shared through fine-grained (coherent) host memory.
//
// Layout and constants are the wire format of include/gfd/descriptor_queue.h:9-53
// in the reference and must stay byte-identical: GPU kernels and the CPU
// poller agree on them, and existing callers size their allocations with
// sizeof(DescriptorQueue).
//
// Ordering protocol on MI355X:
//   producer (wave64 kernel): write the 32-byte body, then a system-scope
//     release store of `sequence = slot + 1`;
//   consumer (CPU poller): acquire-load `sequence`, copy the descriptor,
//     release-store `sequence = 0`, advance `read_idx`;
//   completion: the poller release-stores `done_idx` only after every DMA for
//     slots below it has finished; GPU waiters acquire-load it at system scope.
#include <cstddef>
#include <cstdint>

namespace gfd {

constexpr int QUEUE_SIZE = 16384;
constexpr int MAX_BATCH_SIZE = 8192;
constexpr int BATCH_THRESHOLD = 4096;

// Entries of <= 2 KB flush at the smaller threshold (about 1 MB per batch).
constexpr size_t ADAPTIVE_BATCH_TARGET_BYTES = 1024 * 1024;
constexpr int BATCH_THRESHOLD_SMALL = 1024;

constexpr uint32_t FLAG_NONE = 0;
constexpr uint32_t FLAG_LAST_IN_BATCH = 1;
constexpr uint32_t FLAG_URGENT = 2;

struct alignas(64) Descriptor {
    uint64_t src_addr;           // host source address
    uint64_t dst_addr;           // device destination address
    uint32_t size;               // bytes
    uint32_t flags;              // FLAG_*
    uint64_t user_data;          // caller payload (tile/list id << 32 | index)
    volatile uint64_t sequence;  // slot + 1 when committed, 0 once consumed
};
static_assert(sizeof(Descriptor) == 64, "Descriptor must be 64 bytes");
static_assert(offsetof(Descriptor, sequence) == 32, "sequence follows the 32-byte body");

struct DescriptorQueue {
    Descriptor entries[QUEUE_SIZE];
    volatile uint64_t write_idx;  // next free slot (producers)
    volatile uint64_t read_idx;   // next slot the poller consumes
    volatile uint64_t done_idx;   // every slot below this has landed in HBM
    uint8_t _padding[64 - 24];
};
static_assert(sizeof(DescriptorQueue) == QUEUE_SIZE * 64 + 64, "DescriptorQueue layout");

struct TokenInfo {
    uint64_t cpu_addr;
    uint32_t token_id;
    uint32_t expert_id;
};
static_assert(sizeof(TokenInfo) == 16, "TokenInfo must be 16 bytes");

}  // namespace gfd
