#pragma once
// Tiled-mode device primitives for wave64 HIP kernels on gfx950 (the
// reference's include/gfd/device_primitives.cuh:19-209: acquire_tile,
// acquire_chunk_slots, write_chunk, commit_chunk, wait_chunk_done,
// wait_queue_space, submit_chunk, submit_tile).  Include from HIP sources.
//
// They let a kernel drive the CPU poller's tiled mode itself: a wave claims
// ring slots, writes one descriptor per token of a chunk (user_data =
// tile_id << 32 | token), commits them, and waits until the poller's copies
// have raised the tile's cumulative progress word (d_tile_chunk_done in HBM,
// else tile_chunk_done in host memory).  WarpSpecSession kernels do not need
// them: their transfer waves copy the bytes themselves.
//
// Wave-collective operations are called by all 64 lanes of a wave.  Slot
// claims and tile claims are system-scope atomics on the TiledQueue in
// fine-grained host memory, as the reference's are.  Each lane commits the
// slots it wrote (same lane stride in write and commit), so its release store
// of `sequence` orders its own descriptor body before it.  Every wait is
// bounded and reports whether it was met.
#include <hip/hip_runtime.h>

#include "gfd/device.h"
#include "gfd/tiled_queue.h"

namespace gfd {
namespace device {

__device__ __forceinline__ int wave_lane() { return (int)(threadIdx.x & 63); }

// Next tile id; >= scheduler.total_tiles once every tile is taken.  One lane
// per workgroup calls it and broadcasts the result.
__device__ __forceinline__ uint32_t acquire_tile(TiledQueue* tq) {
    return __hip_atomic_fetch_add(const_cast<uint32_t*>(&tq->scheduler.next_tile), 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_SYSTEM);
}

// Wave-collective: lane 0 claims `count` consecutive ring slots; every lane
// gets the first one.
__device__ __forceinline__ uint64_t acquire_chunk_slots(TiledQueue* tq, uint32_t count) {
    uint64_t base = 0;
    if (wave_lane() == 0)
        base = __hip_atomic_fetch_add(const_cast<uint64_t*>(&tq->base.write_idx), (uint64_t)count, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_SYSTEM);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Descriptor i of the chunk: token tile_id * T + chunk_id * C + i, same byte
// offset on both sides; FLAG_LAST_IN_TILE on the chunk's last entry (the
// poller flushes there) and FLAG_LAST_CHUNK_IN_TILE on the tile's last.
__device__ __forceinline__ void write_chunk(TiledQueue* tq, uint64_t slot_base, uint32_t tile_id, uint32_t chunk_id,
                                            uint32_t tokens_per_chunk, uint32_t tokens_per_tile,
                                            const void* cpu_base, void* gpu_base, uint32_t token_size) {
    const uint32_t C = tokens_per_chunk, T = tokens_per_tile, K = T / C;
    for (uint32_t i = (uint32_t)wave_lane(); i < C; i += 64) {
        const uint32_t g = tile_id * T + chunk_id * C + i;
        uint32_t flags = i == C - 1 ? FLAG_LAST_IN_TILE : FLAG_NONE;
        if (i == C - 1 && chunk_id == K - 1) flags |= FLAG_LAST_CHUNK_IN_TILE;
        const uint64_t off = (uint64_t)g * token_size;
        write_descriptor_raw(&tq->base, slot_base + i, (uint64_t)(uintptr_t)cpu_base + off,
                             (uint64_t)(uintptr_t)gpu_base + off, token_size, flags, ((uint64_t)tile_id << 32) | g);
    }
}

// Wave-collective: publish slots [slot_base, slot_base + count) to the poller.
__device__ __forceinline__ void commit_chunk(TiledQueue* tq, uint64_t slot_base, uint32_t count) {
    for (uint32_t i = (uint32_t)wave_lane(); i < count; i += 64) commit_slot(&tq->base, slot_base + i);
}

// One lane: wait until the tile's cumulative landed-token count reaches
// `expected`.  False after max_ticks of the 100 MHz wall clock.
__device__ __forceinline__ bool wait_chunk_done(TiledQueue* tq, uint32_t tile_id, uint64_t expected,
                                                uint64_t max_ticks = kDefaultWaitTicks) {
    const volatile uint64_t* signal =
        tq->d_tile_chunk_done ? tq->d_tile_chunk_done + tile_id : &tq->tile_chunk_done[tile_id];
    const uint64_t t0 = wall_clock64();
    for (uint32_t n = 0;; n++) {
        if (load_relaxed_system(signal) >= expected) {
            acquire_system();
            return true;
        }
        if (wall_clock64() - t0 > max_ticks) return false;
        if (n >= 64) __builtin_amdgcn_s_sleep(8);
    }
}

// Wave-collective: wait until the ring has room for 2 * needed more slots.
__device__ __forceinline__ bool wait_queue_space(TiledQueue* tq, uint32_t needed,
                                                 uint64_t max_ticks = kDefaultWaitTicks) {
    const uint64_t t0 = wall_clock64();
    bool ok = true;
    for (;;) {
        const uint64_t w = load_relaxed_system(&tq->base.write_idx);
        const uint64_t r = load_relaxed_system(&tq->base.read_idx);
        if (w - r + 2ull * needed <= (uint64_t)QUEUE_SIZE) {
            acquire_system();
            break;
        }
        if (wall_clock64() - t0 > max_ticks) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(8);
    }
    return __builtin_amdgcn_readfirstlane((int)ok) != 0;
}

__device__ __forceinline__ void submit_chunk(TiledQueue* tq, uint64_t slot_base, uint32_t tile_id, uint32_t chunk_id,
                                             uint32_t tokens_per_chunk, uint32_t tokens_per_tile,
                                             const void* cpu_base, void* gpu_base, uint32_t token_size) {
    write_chunk(tq, slot_base, tile_id, chunk_id, tokens_per_chunk, tokens_per_tile, cpu_base, gpu_base, token_size);
    commit_chunk(tq, slot_base, tokens_per_chunk);
}

// Wave-collective: all T descriptors of a tile in one claim and commit;
// FLAG_LAST_IN_TILE on every C-th entry, FLAG_LAST_CHUNK_IN_TILE on the last.
__device__ __forceinline__ void submit_tile(TiledQueue* tq, uint64_t slot_base, uint32_t tile_id, uint32_t T,
                                            uint32_t C, const void* cpu_base, void* gpu_base, uint32_t token_size) {
    for (uint32_t i = (uint32_t)wave_lane(); i < T; i += 64) {
        const uint32_t g = tile_id * T + i;
        uint32_t flags = (i % C) == C - 1 ? FLAG_LAST_IN_TILE : FLAG_NONE;
        if (i == T - 1) flags |= FLAG_LAST_CHUNK_IN_TILE;
        const uint64_t off = (uint64_t)g * token_size;
        write_descriptor_raw(&tq->base, slot_base + i, (uint64_t)(uintptr_t)cpu_base + off,
                             (uint64_t)(uintptr_t)gpu_base + off, token_size, flags, ((uint64_t)tile_id << 32) | g);
    }
    commit_chunk(tq, slot_base, T);
}

}  // namespace device
}  // namespace gfd
