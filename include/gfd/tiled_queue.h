#pragma once
// Tile-scheduled extension of the descriptor ring used by WarpSpecSession.
// Same layout as include/gfd/tiled_queue.h:8-43 of the reference.
#include "gfd/descriptor_queue.h"

namespace gfd {

constexpr int MAX_TILES = 1024;
constexpr uint32_t FLAG_LAST_IN_TILE = 4;        // last entry of a chunk: poller flushes
constexpr uint32_t FLAG_LAST_CHUNK_IN_TILE = 8;  // last entry of a tile

struct alignas(64) TileScheduler {
    volatile uint32_t next_tile;
    uint32_t total_tiles;
    uint32_t tokens_per_tile;
    uint32_t tokens_per_chunk;
    uint32_t chunks_per_tile;
    uint32_t token_size;
    uint8_t _pad[40];
};
static_assert(sizeof(TileScheduler) == 64, "TileScheduler must be 64 bytes");

struct TiledQueue {
    DescriptorQueue base;
    TileScheduler scheduler;
    volatile uint64_t tile_chunk_done[MAX_TILES];  // host-visible cumulative progress
    uint64_t* d_tile_chunk_done;                   // device-memory progress (preferred)
};

// Tile dispatch counter kept in HBM right after d_tile_chunk_done[MAX_TILES]
// (sessions allocate MAX_TILES + TILE_DEVICE_COUNTER_WORDS words), so tile
// claims are device-scope atomics instead of atomics into host memory.
struct TileDeviceCounters {
    uint64_t next_tile;
    uint64_t tiles_done;
    uint64_t error;  // nonzero: a bounded wait gave up (bit flags)
    uint64_t _pad[5];
};
constexpr int TILE_DEVICE_COUNTER_WORDS = (int)(sizeof(TileDeviceCounters) / sizeof(uint64_t));
static_assert(sizeof(TileDeviceCounters) == 64, "TileDeviceCounters is one cache line");

}  // namespace gfd
