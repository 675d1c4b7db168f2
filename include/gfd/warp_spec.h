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
// tiles (device-scope atomic on an HBM counter) and copies the tile's bytes
// straight from pinned host memory to HBM (zero-copy).  Waves after the
// compute waves are transfer helpers: wave 0 and the helpers claim pieces of
// the tile's chunks from an LDS counter, so one workgroup keeps several
// waves' loads in flight over PCIe (one wave alone reaches ~3.3 GB/s, a CU
// ~13 GB/s).  After a device-scope release each piece raises its chunk's
// count in LDS.  Compute wave k (1..K) waits until every piece of chunk k has
// landed (LDS acquire + s_sleep), then runs the functor on it.  The
// double-buffer variant keeps two tile slots with K compute waves each, so the
// transfer of tile n+1 overlaps the compute of tile n.  Blocks are
// 64 * (1 + K + H) (single) or 64 * (1 + 2K + H) (double) threads, at most
// 1024, H helpers.
#include "gfd/tiled_queue.h"
#include "gfd/wave_ops.h"

namespace gfd {
namespace warp_spec {

constexpr int MAX_CHUNKS_PER_TILE = 16;
constexpr uint32_t TILE_END = 0xFFFFFFFFu;
constexpr uint64_t WS_ERR_SLOT_WAIT = 1;
constexpr uint64_t WS_ERR_CHUNK_WAIT = 2;
constexpr uint64_t WS_ERR_HELPER_WAIT = 4;  // transfer waves: a tile's hand-off between them stalled

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
// The d_tile_chunk_done array the counters follow.  tq lives in host memory:
// deriving the array from the counters' address instead of reading
// tq->d_tile_chunk_done again spares a round trip across PCIe per tile.
__device__ __forceinline__ uint64_t* tile_done_words(TileDeviceCounters* cnt) {
    return reinterpret_cast<uint64_t*>(cnt) - MAX_TILES;
}

struct _TileSlot {
    uint32_t tile;  // TILE_END: no more tiles
    int seq;        // n + 1 once the n-th tile of this slot is assigned
    int done;       // chunks whose compute has finished for the current tile
    int chunk_done[MAX_CHUNKS_PER_TILE];  // pieces of chunk k already in HBM
    // Functors with kSplitsChunks: chunk k's token groups, claimed as
    // (epoch << 16 | next token) with epoch = the tile's seq (so a claim can
    // never take a token of the slot's next tile), and tokens computed.
    int claim[MAX_CHUNKS_PER_TILE];
    int toks_done[MAX_CHUNKS_PER_TILE];
};

// A compute functor that declares `static constexpr bool kSplitsChunks =
// true` processes every token on its own (its result for a token does not
// depend on the chunk's other tokens).  Its chunks are then computed in
// groups of tokens by any compute wave: a wave takes its own chunk, then
// helps with the tile's other chunks as they land, and the compute waves of a
// slot left without tiles help finish the other slot's last tile, so the
// compute of a tile's last chunk is not left to one wave after the copy
// ends.  The functor sees each group as a ChunkView of that group's tokens.
// Functors without the declaration see each chunk once, on its own wave, as
// with the reference.
template <typename F, typename = void>
struct _splits_chunks {
    static constexpr bool value = false;
};
template <typename F>
struct _splits_chunks<F, decltype((void)F::kSplitsChunks)> {
    static constexpr bool value = F::kSplitsChunks;
};

// Wait until chunk k of the slot's tile at `epoch` has landed while some of
// its tokens are still unclaimed: 1 (landed, after an acquire), 0 (nothing
// left to claim there: all claimed, or the slot has moved past the epoch), or
// -1 (the bounded wait gave up).
__device__ __forceinline__ int _wait_claimable(_TileSlot& sl, int epoch, uint32_t k, uint32_t P, uint32_t C) {
    for (uint64_t t = 0; t < wave::kSpinLimit; t++) {
        const int c = wave::lds_load(&sl.claim[k]);
        if ((c >> 16) != (epoch & 0x7FFF) || (uint32_t)(c & 0xFFFF) >= C) return 0;
        if (wave::lds_load(&sl.chunk_done[k]) == (int)P) {
            wave::acquire_agent();
            return 1;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return -1;
}

// Claim and compute token groups (G tokens) of chunk k of `tile`, the tile of
// slot `sl` at epoch `epoch` (its seq), until none is left.  The chunk must
// have landed (the caller saw chunk_done[k] == P and made an acquire).  The
// group that completes the chunk counts it in `done`.
template <typename ComputeFn>
__device__ __forceinline__ void _compute_groups(_TileSlot& sl, int epoch, uint32_t tile, uint32_t k, uint32_t T,
                                                uint32_t C, uint32_t G, uint32_t token_size, void* gpu_buffer,
                                                ComputeFn& compute_fn) {
    const int lane = wave::lane_id();
    for (;;) {
        // The retry loop is wave-uniform and only the compare-and-swap is
        // lane 0's: the functor then runs with every lane active.  (A retry
        // loop inside lane 0's branch left the functor's cross-lane sums
        // wrong on every group after a wave's first.)
        const int w = __builtin_amdgcn_readfirstlane(wave::lds_load(&sl.claim[k]));
        if ((w >> 16) != (epoch & 0x7FFF) || (uint32_t)(w & 0xFFFF) >= C) return;
        bool won = false;
        if (lane == 0) {
            int expect = w;
            won = __hip_atomic_compare_exchange_strong(&sl.claim[k], &expect, w + (int)G, __ATOMIC_ACQ_REL,
                                                       __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (__ballot(won) == 0) continue;
        const int got = w & 0xFFFF;
        const uint32_t n = C - (uint32_t)got < G ? C - (uint32_t)got : G;
        ChunkView v;
        v.global_token_offset = tile * T + k * C + (uint32_t)got;
        v.base_ptr = (char*)gpu_buffer + (uint64_t)v.global_token_offset * token_size;
        v.token_size = token_size;
        v.size = n;
        v.tile_id = tile;
        v.chunk_id = k;
        v.lane_id = lane;
        compute_fn(v);
        if (lane == 0) {
            const int before =
                __hip_atomic_fetch_add(&sl.toks_done[k], (int)n, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
            if ((uint32_t)before + n == C) wave::lds_add(&sl.done, 1);
        }
    }
}

// The tile the transfer waves copy together: wave 0 publishes it, every
// transfer wave claims its pieces, each helper acknowledges it (even with no
// piece left to claim) and only then is the next tile published, so no helper
// reads a job's fields while they change.
struct _TileJob {
    uint32_t tile;
    int slot;
    int seq;         // n + 1 once the n-th job is published; -1: no more jobs
    int next_piece;  // pieces claimed
    int pieces_done;
    int acks;        // helpers finished with this job
};

// Pieces per chunk: enough that every transfer wave has one when a tile has
// fewer chunks than transfer waves, none under 16 KiB.
__device__ __forceinline__ uint32_t _pieces_per_chunk(uint32_t K, uint32_t transfer_waves, uint64_t chunk_bytes) {
    uint32_t p = (transfer_waves + K - 1) / K;
    const uint64_t pmax = chunk_bytes / 16384;
    if ((uint64_t)p > pmax) p = pmax > 0 ? (uint32_t)pmax : 1u;
    return p;
}

// Claim and copy pieces of the current job (tile, slot); returns the pieces
// copied.  The caller passes the job's fields in registers: wave 0 has them
// from its own claim, a helper read them after every lane's acquire of
// job->seq.  (Lanes 1..63 of wave 0 must not read them back from LDS: lane
// 0's plain stores there are not ordered before other lanes' loads, and the
// compiler does schedule such loads ahead of the stores.)
__device__ __forceinline__ int _copy_pieces(_TileJob* job, _TileSlot* slots, uint64_t tile, int slot_idx, uint32_t K,
                                            uint32_t P, uint64_t chunk_bytes, uint64_t piece_bytes, uint32_t T,
                                            uint32_t C, uint32_t token_size, void* gpu_buffer, const void* cpu_base,
                                            int unroll) {
    const int lane = wave::lane_id();
    _TileSlot& slot = slots[slot_idx];
    int mine = 0;
    for (;;) {
        int i = 0;
        if (lane == 0) i = __hip_atomic_fetch_add(&job->next_piece, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        i = __builtin_amdgcn_readfirstlane(i);
        if ((uint32_t)i >= K * P) break;
        const uint32_t k = (uint32_t)i / P, j = (uint32_t)i % P;
        const uint64_t begin = (uint64_t)j * piece_bytes;
        const uint64_t n = begin < chunk_bytes ? (chunk_bytes - begin < piece_bytes ? chunk_bytes - begin : piece_bytes) : 0;
        const uint64_t off = (tile * T + (uint64_t)k * C) * token_size + begin;
        if (n) wave::copy_u(unroll, (uint64_t)(uintptr_t)gpu_buffer + off, (uint64_t)(uintptr_t)cpu_base + off, n);
        wave::release_agent();  // the piece is visible device-wide before the compute wave hears of it
        if (lane == 0) wave::lds_add(&slot.chunk_done[k], 1);
        mine++;
    }
    return mine;
}

template <int NSLOTS, typename ComputeFn>
__device__ __forceinline__ void _tile_loop(TiledQueue* tq, void* gpu_buffer, const void* cpu_base, ComputeFn compute_fn) {
    __shared__ _TileSlot slots[NSLOTS];
    __shared__ _TileJob job;
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
        slots[threadIdx.x].done = (int)K;  // free
        slots[threadIdx.x].tile = 0;
        for (int k = 0; k < MAX_CHUNKS_PER_TILE; k++) {
            slots[threadIdx.x].claim[k] = (int)C;  // epoch 0: nothing to claim
            slots[threadIdx.x].toks_done[k] = 0;
        }
    }
    if (threadIdx.x == 0) job.seq = 0;
    __syncthreads();

    // Waves after the compute waves are transfer helpers.
    const int nwaves = (int)(blockDim.x / wave::kWidth);
    const int first_helper = 1 + NSLOTS * (int)K;
    const int helpers = nwaves > first_helper ? nwaves - first_helper : 0;
    const uint64_t chunk_bytes = (uint64_t)C * token_size;
    const uint32_t P = _pieces_per_chunk(K, 1u + (uint32_t)helpers, chunk_bytes);
    const uint64_t piece_bytes = ((chunk_bytes + P - 1) / P + 1023) & ~1023ull;
    const uint32_t active = gridDim.x < total_tiles ? gridDim.x : total_tiles;
    const int unroll = wave::transfer_unroll(active * (1u + (uint32_t)helpers));

    if (w == 0) {
        // ---------------- transfer wave (leader)
        for (uint32_t n = 0;; n++) {
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
                const int epoch = (int)(n / NSLOTS) + 1;
                slots[s].tile = last ? TILE_END : (uint32_t)tile;
                for (uint32_t k = 0; k < K; k++) {
                    slots[s].chunk_done[k] = 0;
                    if (!last) {
                        slots[s].claim[k] = (epoch & 0x7FFF) << 16;
                        slots[s].toks_done[k] = 0;
                    }
                }
                slots[s].done = 0;
                wave::lds_store(&slots[s].seq, epoch);
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
            if (lane == 0) {
                job.tile = (uint32_t)tile;
                job.slot = s;
                job.next_piece = 0;
                job.pieces_done = 0;
                job.acks = 0;
                wave::lds_store(&job.seq, (int)n + 1);
            }
            const int mine = _copy_pieces(&job, slots, tile, s, K, P, chunk_bytes, piece_bytes, T, C, token_size,
                                          gpu_buffer, cpu_base, unroll);
            if (lane == 0) wave::lds_add(&job.pieces_done, mine);
            if (helpers > 0 &&
                (!wave::wait_lds_eq(&job.pieces_done, (int)(K * P)) || !wave::wait_lds_eq(&job.acks, helpers))) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, WS_ERR_HELPER_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if (lane == 0) {
                if (tile < (uint64_t)MAX_TILES)
                    __hip_atomic_store(&tile_done_words(cnt)[tile], (uint64_t)T, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(&cnt->tiles_done, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (lane == 0) wave::lds_store(&job.seq, -1);  // helpers exit
    } else if (w >= first_helper) {
        // ---------------- transfer helper: copies pieces of the leader's tiles
        for (int want = 1;;) {
            int seq = 0;
            bool ok = false;
            for (uint64_t i = 0; i < wave::kSpinLimit; i++) {
                seq = wave::lds_load(&job.seq);
                if (seq < 0 || seq >= want) {
                    ok = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (!ok) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, WS_ERR_HELPER_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if (seq < 0) break;
            const int mine = _copy_pieces(&job, slots, job.tile, job.slot, K, P, chunk_bytes, piece_bytes, T, C,
                                          token_size, gpu_buffer, cpu_base, unroll);
            if (lane == 0) {
                wave::lds_add(&job.pieces_done, mine);
                wave::lds_add(&job.acks, 1);
            }
            want = seq + 1;
        }
    } else if ((uint32_t)(w - 1) < NSLOTS * K && _splits_chunks<ComputeFn>::value) {
        // ---------------- compute waves sharing the chunks: slot g, chunk k first
        const int g = (int)((uint32_t)(w - 1) / K);
        const uint32_t k = (uint32_t)(w - 1) % K;
        uint32_t G = C / (NSLOTS * K);
        G = G ? G : 1u;
        for (int n = 1;; n++) {
            if (!wave::wait_lds_eq(&slots[g].seq, n)) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, WS_ERR_CHUNK_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            const uint32_t tile = slots[g].tile;
            if (tile == TILE_END) {
                // No more tiles for this slot: help with the other slot's
                // tile while it is still the same one.
                for (int o = 1; o < NSLOTS; o++) {
                    _TileSlot& other = slots[(g + o) % NSLOTS];
                    const int epoch = wave::lds_load(&other.seq);
                    const uint32_t otile = other.tile;
                    if (epoch == 0 || otile == TILE_END) continue;
                    for (uint32_t i = 0; i < K; i++) {
                        const uint32_t k2 = (k + i) % K;
                        const int r = _wait_claimable(other, epoch, k2, P, C);
                        if (r < 0) break;  // its own waves report a stall
                        if (r > 0) _compute_groups(other, epoch, otile, k2, T, C, G, token_size, gpu_buffer, compute_fn);
                    }
                }
                break;
            }
            // This wave's chunk, then the tile's later chunks as they land,
            // then the earlier ones, each while tokens are left to claim (the
            // slot is refilled only once all of the tile's chunks are done,
            // so waiting here costs nothing).
            bool ok = true;
            for (uint32_t i = 0; i < K && ok; i++) {
                const uint32_t k2 = (k + i) % K;
                const int r = _wait_claimable(slots[g], n, k2, P, C);
                if (r < 0) {
                    if (lane == 0) __hip_atomic_fetch_or(&cnt->error, WS_ERR_CHUNK_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = false;
                } else if (r > 0) {
                    _compute_groups(slots[g], n, tile, k2, T, C, G, token_size, gpu_buffer, compute_fn);
                }
            }
            if (!ok) break;
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
            if (!wave::wait_lds_eq(&slots[g].chunk_done[k], (int)P)) {
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
