#pragma once
// Wave-specialised tile framework (HIP sources only).  Same kernel interface
// as the reference's include/gfd/warp_spec.cuh:41-469:
//
//   struct MyCompute { __device__ void operator()(gfd::warp_spec::ChunkView c) { ... } };
//   GFD_WARP_SPEC_KERNEL(my_kernel, MyCompute);     // (TiledQueue*, void* gpu_dst, const void* cpu_src, MyCompute)
//   GFD_WARP_SPEC_KERNEL_DB(my_kernel_db, MyCompute);
//
// Work: tile t = tokens [t*T, (t+1)*T) of a linear token range, cut into K
// chunks of C tokens.  Wave 0 of a workgroup is the transfer wave: it claims
// tiles (device-scope atomic on an HBM counter), copies each chunk's bytes
// straight from pinned host memory to HBM (zero-copy) and raises the chunk
// count in LDS after a device-scope release.  Compute wave k (1..K) waits for
// chunk k (LDS acquire + s_sleep), then runs the functor on it.  The
// double-buffer variant keeps two tile slots with K compute waves each, so the
// transfer of tile n+1 overlaps the compute of tile n.  Blocks are
// 64 * (1 + K) (single) or 64 * (1 + 2K) (double) threads, at most 1024.
#include "gfd/tiled_queue.h"
#include "gfd/wave_ops.h"

namespace gfd {
namespace warp_spec {

constexpr int MAX_CHUNKS_PER_TILE = 16;
constexpr uint32_t TILE_END = 0xFFFFFFFFu;
constexpr uint64_t WS_ERR_SLOT_WAIT = 1;
constexpr uint64_t WS_ERR_CHUNK_WAIT = 2;

// Read-only view of a chunk whose data is in HBM.
struct ChunkView {
    void* base_ptr;
    uint32_t token_size;
    uint32_t size;  // tokens in this chunk
    uint32_t tile_id;
    uint32_t chunk_id;
    uint32_t global_token_offset;
    int lane_id;

    template <typename T>
    __device__ __forceinline__ T* data(int local_token_idx) const {
        return reinterpret_cast<T*>((char*)base_ptr + (uint64_t)local_token_idx * token_size);
    }
    __device__ __forceinline__ int global_idx(int local_token_idx) const {
        return (int)global_token_offset + local_token_idx;
    }
};

struct TileContext {
    uint32_t tile_id;
    uint32_t tokens_per_tile;
    uint32_t chunks_per_tile;
    uint32_t tokens_per_chunk;
    void* tile_base_ptr;
    uint32_t token_size;

    __device__ __forceinline__ ChunkView get_chunk(int chunk_id) const {
        ChunkView v;
        v.base_ptr = (char*)tile_base_ptr + (uint64_t)chunk_id * tokens_per_chunk * token_size;
        v.token_size = token_size;
        v.size = tokens_per_chunk;
        v.tile_id = tile_id;
        v.chunk_id = (uint32_t)chunk_id;
        v.global_token_offset = tile_id * tokens_per_tile + (uint32_t)chunk_id * tokens_per_chunk;
        v.lane_id = wave::lane_id();
        return v;
    }
};

__device__ __forceinline__ TileDeviceCounters* tile_counters(TiledQueue* tq) {
    return reinterpret_cast<TileDeviceCounters*>(tq->d_tile_chunk_done + MAX_TILES);
}

struct _TileSlot {
    uint32_t tile;  // TILE_END: no more tiles
    int seq;        // n + 1 once the n-th tile of this slot is assigned
    int ready;      // chunks of the current tile already in HBM
    int done;       // compute waves finished with the current tile
};

template <int NSLOTS, typename ComputeFn>
__device__ __forceinline__ void _tile_loop(TiledQueue* tq, void* gpu_buffer, const void* cpu_base, ComputeFn compute_fn) {
    __shared__ _TileSlot slots[NSLOTS];
    const int w = wave::wave_id();
    const int lane = wave::lane_id();
    const uint32_t C = tq->scheduler.tokens_per_chunk;
    const uint32_t K = tq->scheduler.chunks_per_tile;
    const uint32_t T = tq->scheduler.tokens_per_tile;
    const uint32_t total_tiles = tq->scheduler.total_tiles;
    const uint32_t token_size = tq->scheduler.token_size;
    TileDeviceCounters* cnt = tile_counters(tq);
    if (threadIdx.x < NSLOTS) {
        slots[threadIdx.x].seq = 0;
        slots[threadIdx.x].ready = 0;
        slots[threadIdx.x].done = (int)K;  // free
        slots[threadIdx.x].tile = 0;
    }
    __syncthreads();

    if (w == 0) {
        // ---------------- transfer wave
        const int unroll = wave::transfer_unroll(gridDim.x < total_tiles ? gridDim.x : total_tiles);
        bool ok = true;
        for (uint32_t n = 0; ok; n++) {
            const int s = (int)(n % NSLOTS);
            if (!wave::wait_lds_eq(&slots[s].done, (int)K)) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, WS_ERR_SLOT_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            uint64_t tile = 0;
            if (lane == 0) tile = __hip_atomic_fetch_add(&cnt->next_tile, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            tile = wave::broadcast0(tile);
            const bool last = tile >= total_tiles;
            if (lane == 0) {
                slots[s].tile = last ? TILE_END : (uint32_t)tile;
                slots[s].ready = 0;
                slots[s].done = 0;
                wave::lds_store(&slots[s].seq, (int)(n / NSLOTS) + 1);
            }
            if (last) {
                // Hand TILE_END to the other slot(s) as well, once they are free.
                for (int o = 1; o < NSLOTS; o++) {
                    const int so = (int)((n + o) % NSLOTS);
                    if (!wave::wait_lds_eq(&slots[so].done, (int)K)) break;
                    if (lane == 0) {
                        slots[so].tile = TILE_END;
                        slots[so].done = 0;
                        wave::lds_store(&slots[so].seq, (int)((n + o) / NSLOTS) + 1);
                    }
                }
                break;
            }
            const uint64_t tok0 = tile * T;
            for (uint32_t k = 0; k < K; k++) {
                const uint64_t off = (tok0 + (uint64_t)k * C) * token_size;
                wave::copy_u(unroll, (uint64_t)(uintptr_t)gpu_buffer + off, (uint64_t)(uintptr_t)cpu_base + off,
                             (uint64_t)C * token_size);
                wave::release_agent();
                if (lane == 0) wave::lds_store(&slots[s].ready, (int)k + 1);
            }
            if (lane == 0) {
                if (tile < (uint64_t)MAX_TILES)
                    __hip_atomic_store(&tq->d_tile_chunk_done[tile], (uint64_t)T, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(&cnt->tiles_done, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    } else if ((uint32_t)(w - 1) < NSLOTS * K) {
        // ---------------- compute waves: slot g, chunk k
        const int g = (int)((uint32_t)(w - 1) / K);
        const uint32_t k = (uint32_t)(w - 1) % K;
        for (int n = 1;; n++) {
            if (!wave::wait_lds_eq(&slots[g].seq, n)) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, WS_ERR_CHUNK_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            const uint32_t tile = slots[g].tile;
            if (tile == TILE_END) break;
            if (!wave::wait_lds_gt(&slots[g].ready, (int)k)) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, WS_ERR_CHUNK_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            wave::acquire_agent();
            ChunkView v;
            v.global_token_offset = tile * T + k * C;
            v.base_ptr = (char*)gpu_buffer + (uint64_t)v.global_token_offset * token_size;
            v.token_size = token_size;
            v.size = C;
            v.tile_id = tile;
            v.chunk_id = k;
            v.lane_id = lane;
            compute_fn(v);
            if (lane == 0) wave::lds_add(&slots[g].done, 1);
        }
    }
}

template <typename ComputeFn>
__device__ __forceinline__ void _warp_spec_tile_loop(TiledQueue* tq, void* gpu_buffer, const void* cpu_base, ComputeFn fn) {
    _tile_loop<1>(tq, gpu_buffer, cpu_base, fn);
}

template <typename ComputeFn>
__device__ __forceinline__ void _warp_spec_tile_loop_double_buffer(TiledQueue* tq, void* gpu_buffer, const void* cpu_base,
                                                   ComputeFn fn) {
    _tile_loop<2>(tq, gpu_buffer, cpu_base, fn);
}

}  // namespace warp_spec
}  // namespace gfd

#define GFD_WARP_SPEC_KERNEL(kernel_name, ComputeFnType)                                        \
    __global__ void kernel_name(gfd::TiledQueue* tq, void* gpu_buffer, const void* cpu_base,   \
                                ComputeFnType compute_fn) {                                     \
        gfd::warp_spec::_warp_spec_tile_loop(tq, gpu_buffer, cpu_base, compute_fn);             \
    }

#define GFD_WARP_SPEC_KERNEL_DB(kernel_name, ComputeFnType)                                     \
    __global__ void kernel_name(gfd::TiledQueue* tq, void* gpu_buffer, const void* cpu_base,   \
                                ComputeFnType compute_fn) {                                     \
        gfd::warp_spec::_warp_spec_tile_loop_double_buffer(tq, gpu_buffer, cpu_base, compute_fn); \
    }
