// The CPU poller's tiled mode driven from a kernel with the tiled device
// primitives (include/gfd/device_primitives.h): the reference's per-tile
// baseline of examples/07_warp_spec_simple.cu:88-134 (baseline_kernel), one
// workgroup per tile.  Wave 0 claims ring slots and submits the tile chunk by
// chunk (or whole), waiting for the poller's per-tile progress word after
// each; then the workgroup reads the landed tokens and writes each token's
// u32-word checksum (an exact integer result).  Also the C-ABI that allocates
// and resets a TiledQueue for it.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstring>

#include "gfd/device_primitives.h"
#include "gfd/tiled_queue.h"
#include "gfd_capi.h"

// Offsets the Python binding reads (gfd_amd.TiledQueue).
static_assert(offsetof(gfd::TiledQueue, scheduler) == sizeof(gfd::DescriptorQueue), "TiledQueue layout");
static_assert(offsetof(gfd::TiledQueue, tile_chunk_done) == sizeof(gfd::DescriptorQueue) + 64, "TiledQueue layout");
static_assert(offsetof(gfd::TiledQueue, d_tile_chunk_done) ==
                  sizeof(gfd::DescriptorQueue) + 64 + 8 * gfd::MAX_TILES, "TiledQueue layout");

namespace {

__global__ __launch_bounds__(256) void tiled_poller_kernel(gfd::TiledQueue* tq, const void* cpu_base, void* gpu_base,
                                                           int whole_tile, uint64_t max_ticks,
                                                           unsigned long long* __restrict__ sums, int* status) {
    __shared__ int ok;
    const uint32_t T = tq->scheduler.tokens_per_tile, C = tq->scheduler.tokens_per_chunk;
    const uint32_t K = tq->scheduler.chunks_per_tile, ts = tq->scheduler.token_size;
    const uint32_t tile = blockIdx.x;
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63), nwaves = (int)(blockDim.x >> 6);
    if (threadIdx.x == 0) ok = 1;
    __syncthreads();
    if (wave == 0) {
        if (whole_tile) {
            const uint64_t base = gfd::device::acquire_chunk_slots(tq, T);
            gfd::device::submit_tile(tq, base, tile, T, C, cpu_base, gpu_base, ts);
            if (lane == 0 && !gfd::device::wait_chunk_done(tq, tile, T, max_ticks)) ok = 0;
        } else {
            for (uint32_t k = 0; k < K; k++) {
                const uint64_t base = gfd::device::acquire_chunk_slots(tq, C);
                gfd::device::submit_chunk(tq, base, tile, k, C, T, cpu_base, gpu_base, ts);
                int landed = 1;
                if (lane == 0) landed = gfd::device::wait_chunk_done(tq, tile, (uint64_t)(k + 1) * C, max_ticks);
                if (!__builtin_amdgcn_readfirstlane(landed)) {
                    if (lane == 0) ok = 0;
                    break;
                }
            }
        }
    }
    __syncthreads();
    if (!ok) {
        if (threadIdx.x == 0) __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return;
    }
    // The copy engines wrote the tokens: every lane acquires before reading.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
    const uint32_t nw = ts / 4;
    for (uint32_t j = (uint32_t)wave; j < T; j += (uint32_t)nwaves) {
        const uint64_t g = (uint64_t)tile * T + j;
        const uint8_t* p = (const uint8_t*)gpu_base + g * ts;
        unsigned long long acc = 0;
        if (((uintptr_t)p & 3) == 0) {
            const uint32_t* w = (const uint32_t*)p;
            for (uint32_t i = (uint32_t)lane; i < nw; i += 64) acc += w[i];
        } else {
            for (uint32_t i = (uint32_t)lane; i < nw; i += 64)
                acc += (uint32_t)p[4 * i] | ((uint32_t)p[4 * i + 1] << 8) | ((uint32_t)p[4 * i + 2] << 16) |
                       ((uint32_t)p[4 * i + 3] << 24);
        }
        for (uint32_t b = nw * 4 + (uint32_t)lane; b < ts; b += 64) acc += p[b];
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)acc, o, 64);
            const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(acc >> 32), o, 64);
            acc += ((unsigned long long)hi << 32) | lo;
        }
        if (lane == 0) sums[g] = acc;
    }
}

}  // namespace

extern "C" int gfd_tiled_queue_alloc(void** out, uint32_t total_tiles, uint32_t tokens_per_tile,
                                     uint32_t tokens_per_chunk, uint32_t token_size, int device_signals) {
    if (!out || total_tiles == 0 || total_tiles > (uint32_t)gfd::MAX_TILES || tokens_per_chunk == 0 ||
        tokens_per_tile == 0 || tokens_per_tile % tokens_per_chunk != 0 || token_size == 0)
        return (int)hipErrorInvalidValue;
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, sizeof(gfd::TiledQueue), hipHostMallocCoherent);
    if (e != hipSuccess) return (int)e;
    std::memset(p, 0, sizeof(gfd::TiledQueue));
    auto* tq = static_cast<gfd::TiledQueue*>(p);
    tq->scheduler.total_tiles = total_tiles;
    tq->scheduler.tokens_per_tile = tokens_per_tile;
    tq->scheduler.tokens_per_chunk = tokens_per_chunk;
    tq->scheduler.chunks_per_tile = tokens_per_tile / tokens_per_chunk;
    tq->scheduler.token_size = token_size;
    if (device_signals) {
        void* d = nullptr;
        e = hipMalloc(&d, sizeof(uint64_t) * gfd::MAX_TILES);
        if (e == hipSuccess) e = hipMemset(d, 0, sizeof(uint64_t) * gfd::MAX_TILES);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            if (d) (void)hipFree(d);
            (void)hipHostFree(p);
            return (int)e;
        }
        tq->d_tile_chunk_done = static_cast<uint64_t*>(d);
    }
    *out = p;
    return 0;
}

extern "C" int gfd_tiled_queue_free(void* p) {
    if (!p) return 0;
    auto* tq = static_cast<gfd::TiledQueue*>(p);
    if (tq->d_tile_chunk_done) (void)hipFree(tq->d_tile_chunk_done);
    return (int)hipHostFree(p);
}

extern "C" int gfd_tiled_queue_reset(void* p) {
    if (!p) return (int)hipErrorInvalidValue;
    auto* tq = static_cast<gfd::TiledQueue*>(p);
    std::memset((void*)&tq->base, 0, sizeof(tq->base));
    std::memset((void*)tq->tile_chunk_done, 0, sizeof(tq->tile_chunk_done));
    tq->scheduler.next_tile = 0;
    if (tq->d_tile_chunk_done) {
        hipError_t e = hipMemset(tq->d_tile_chunk_done, 0, sizeof(uint64_t) * gfd::MAX_TILES);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) return (int)e;
    }
    __atomic_thread_fence(__ATOMIC_SEQ_CST);
    return 0;
}

extern "C" int gfd_tiled_poller_run(void* p, const void* cpu_base, void* gpu_base, int whole_tile,
                                    uint64_t timeout_us, unsigned long long* sums, int* status, void* stream) {
    if (!p || !cpu_base || !gpu_base || !sums || !status) return (int)hipErrorInvalidValue;
    auto* tq = static_cast<gfd::TiledQueue*>(p);
    const uint64_t tokens = (uint64_t)tq->scheduler.total_tiles * tq->scheduler.tokens_per_tile;
    const uint64_t used = tq->base.write_idx - tq->base.read_idx;
    // Slots are claimed without waiting for room: the whole launch must fit the ring.
    if (tq->scheduler.total_tiles == 0 || tokens + used > (uint64_t)gfd::QUEUE_SIZE) return (int)hipErrorInvalidValue;
    const uint64_t ticks = timeout_us * (gfd::device::kWallClockHz / 1000000ull);
    hipLaunchKernelGGL(tiled_poller_kernel, dim3(tq->scheduler.total_tiles), dim3(256), 0, (hipStream_t)stream, tq,
                       cpu_base, gpu_base, whole_tile, ticks, sums, status);
    return (int)hipGetLastError();
}
