// Zero-copy scattered gather for gfx950 (MI355X): wave64 kernels read
// scattered tokens straight out of pinned host memory over PCIe and write them
// contiguously to HBM.  No reference counterpart: the reference always copies
// through CPU staging + copy engines; this is the GPU-initiated alternative
// for the same contract (dst[j*T + b] = token_j[b]).
//
// Memory-level design
//   * Each lane moves 16 bytes per load (global_load_dwordx4); a wave covers
//     1 KiB of one token per instruction, so every PCIe read request is a
//     full, contiguous cache-line group.
//   * Each lane keeps U = 4 independent 16-byte loads in flight before it
//     stores, and the grid is 2 workgroups per CU (512 on MI355X) looping over
//     the data: 512 x 256 x 4 x 16 B = 8 MiB of host reads can be outstanding,
//     far above the link's bandwidth-latency product (about 64 GB/s x 2 us).
//     More concurrency is slower, not faster: with 16 workgroups per CU the
//     kernel drops from 56 to 52 GB/s, because many more distinct host pages
//     are in flight at once (measured over 0.5-32 workgroups per CU and
//     U = 1-16; 2 and 4 are the optimum for 512 B - 64 KiB tokens).
//   * Stores are plain 16-byte stores to HBM (coalesced, contiguous).
//   * Token source addresses come from a per-token table (the KV block/page
//     table), normally resident in HBM; lanes of one token read the same
//     8-byte entry, which the L1/L2 broadcast.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gfd_capi.h"

namespace {

constexpr int kBlock = 256;  // 4 waves

// Byte-wise fallback for a 16-byte vector whose host source is not 16-byte
// aligned (never taken for the benchmark layouts, kept for correctness).
__device__ __forceinline__ uint4 load16_unaligned(const uint8_t* p) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        w[i] = (uint32_t)p[4 * i] | ((uint32_t)p[4 * i + 1] << 8) | ((uint32_t)p[4 * i + 2] << 16) |
               ((uint32_t)p[4 * i + 3] << 24);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ uint4 load16(uint64_t addr) {
    if ((addr & 15) == 0) return *reinterpret_cast<const uint4*>(addr);
    return load16_unaligned(reinterpret_cast<const uint8_t*>(addr));
}

// Page-table form: token j lives at src_addrs[j] (host), lands at
// dst + j * token_size.  token_size is a multiple of 16; the flattened
// 16-byte vector index v = j * vpt + o is split with a shift when vpt is a
// power of two.
template <int U>
__global__ __launch_bounds__(kBlock) void zc_gather_tokens16(const uint64_t* __restrict__ src_addrs,
                                                             uint4* __restrict__ dst, uint32_t vpt,
                                                             int vpt_shift, uint32_t total_vecs) {
    const uint32_t tid = threadIdx.x;
    const uint32_t step = gridDim.x * (uint32_t)(kBlock * U);
    for (uint32_t base = blockIdx.x * (uint32_t)(kBlock * U); base < total_vecs; base += step) {
        uint4 r[U];
#pragma unroll
        for (int k = 0; k < U; k++) {
            const uint32_t v = base + (uint32_t)k * kBlock + tid;
            if (v < total_vecs) {
                uint32_t j, o;
                if (vpt_shift >= 0) {
                    j = v >> vpt_shift;
                    o = v & (vpt - 1);
                } else {
                    j = v / vpt;
                    o = v - j * vpt;
                }
                r[k] = load16(src_addrs[j] + (uint64_t)o * 16u);
            }
        }
#pragma unroll
        for (int k = 0; k < U; k++) {
            const uint32_t v = base + (uint32_t)k * kBlock + tid;
            if (v < total_vecs) dst[v] = r[k];
        }
    }
}

// Page-table form for token sizes that are not a multiple of 16: byte lanes.
__global__ __launch_bounds__(kBlock) void zc_gather_tokens1(const uint64_t* __restrict__ src_addrs,
                                                            uint8_t* __restrict__ dst, uint32_t token_size,
                                                            uint64_t total_bytes) {
    const uint64_t step = (uint64_t)gridDim.x * kBlock;
    for (uint64_t b = (uint64_t)blockIdx.x * kBlock + threadIdx.x; b < total_bytes; b += step) {
        const uint64_t j = b / token_size;
        const uint64_t o = b - j * token_size;
        dst[b] = *reinterpret_cast<const uint8_t*>(src_addrs[j] + o);
    }
}

__device__ __forceinline__ uint64_t readlane64(uint64_t x, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

// Copy one entry with the whole wave.
template <int U>
__device__ __forceinline__ void wave_copy(uint64_t d, uint64_t s, uint64_t n, uint32_t lane) {
    if (((d ^ s) & 15) == 0) {
        // Head bytes up to 16-byte alignment, 16-byte body, tail bytes.
        uint64_t head = (16 - (d & 15)) & 15;
        if (head > n) head = n;
        if (lane < head) *reinterpret_cast<uint8_t*>(d + lane) = *reinterpret_cast<const uint8_t*>(s + lane);
        d += head;
        s += head;
        n -= head;
        const uint64_t nv = n >> 4;
        const uint4* sv = reinterpret_cast<const uint4*>(s);
        uint4* dv = reinterpret_cast<uint4*>(d);
        for (uint64_t base = 0; base < nv; base += 64u * U) {
            uint4 r[U];
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint64_t v = base + (uint64_t)k * 64u + lane;
                if (v < nv) r[k] = sv[v];
            }
#pragma unroll
            for (int k = 0; k < U; k++) {
                const uint64_t v = base + (uint64_t)k * 64u + lane;
                if (v < nv) dv[v] = r[k];
            }
        }
        const uint64_t tail = n & 15;
        if (lane < tail)
            *reinterpret_cast<uint8_t*>(d + (nv << 4) + lane) =
                *reinterpret_cast<const uint8_t*>(s + (nv << 4) + lane);
    } else {
        for (uint64_t b = lane; b < n; b += 64)
            *reinterpret_cast<uint8_t*>(d + b) = *reinterpret_cast<const uint8_t*>(s + b);
    }
}

// Generic SG list: any sizes, any (disjoint) destinations.  Each wave takes
// `per_wave` consecutive entries; lane i loads entry i's 24-byte descriptor
// once and the wave walks them with readlane (one table round trip per batch).
template <int U>
__global__ __launch_bounds__(kBlock) void zc_gather_sg(const gfd_sg_entry* __restrict__ entries, int count,
                                                       int per_wave) {
    const uint32_t lane = threadIdx.x & 63;
    const int wave = (int)((blockIdx.x * kBlock + threadIdx.x) >> 6);
    const int nwaves = (int)((gridDim.x * kBlock) >> 6);
    for (int first = wave * per_wave; first < count; first += nwaves * per_wave) {
        const int n = min(per_wave, count - first);
        uint64_t md = 0, ms = 0, mn = 0;
        if ((int)lane < n) {
            const gfd_sg_entry e = entries[first + lane];
            md = e.dst;
            ms = e.src;
            mn = e.size;
        }
        for (int i = 0; i < n; i++)
            wave_copy<U>(readlane64(md, i), readlane64(ms, i), readlane64(mn, i), lane);
    }
}

int g_cu_count = 0;

int cu_count() {
    if (g_cu_count == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&g_cu_count, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            g_cu_count <= 0)
            g_cu_count = 256;
    }
    return g_cu_count;
}

constexpr int kUnroll = 4;
constexpr int kBlocksPerCU = 2;

}  // namespace

extern "C" int gfd_zero_copy_gather_tokens(const uint64_t* src_addrs, void* dst, uint32_t token_size,
                                           int num_tokens, void* stream) {
    if (num_tokens < 0 || (num_tokens > 0 && (!src_addrs || !dst || token_size == 0)))
        return (int)hipErrorInvalidValue;
    if (num_tokens == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const uint64_t total = (uint64_t)num_tokens * token_size;
    const int max_blocks = cu_count() * kBlocksPerCU;
    if ((token_size & 15) == 0 && ((uintptr_t)dst & 15) == 0) {
        const uint64_t total_vecs = total >> 4;
        if (total_vecs >= (1ull << 31)) return (int)hipErrorInvalidValue;  // >= 32 GiB per call
        const uint32_t vpt = token_size >> 4;
        const int shift = (vpt & (vpt - 1)) == 0 ? __builtin_ctz(vpt) : -1;
        uint64_t blocks = (total_vecs + kBlock * kUnroll - 1) / (kBlock * kUnroll);
        if (blocks > (uint64_t)max_blocks) blocks = max_blocks;
        hipLaunchKernelGGL(zc_gather_tokens16<kUnroll>, dim3((uint32_t)blocks), dim3(kBlock), 0, st, src_addrs,
                           (uint4*)dst, vpt, shift, (uint32_t)total_vecs);
    } else {
        uint64_t blocks = (total + kBlock - 1) / kBlock;
        if (blocks > (uint64_t)max_blocks) blocks = max_blocks;
        hipLaunchKernelGGL(zc_gather_tokens1, dim3((uint32_t)blocks), dim3(kBlock), 0, st, src_addrs,
                           (uint8_t*)dst, token_size, total);
    }
    return (int)hipGetLastError();
}

extern "C" int gfd_zero_copy_gather(const gfd_sg_entry* entries, int count, void* stream) {
    if (count < 0 || (count > 0 && !entries)) return (int)hipErrorInvalidValue;
    if (count == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    // One wave per entry batch, about 4 * 2 waves per CU in flight (the same
    // concurrency as the page-table kernel); at most 64 entries per batch.
    const int max_blocks = cu_count() * kBlocksPerCU;
    const int target_waves = max_blocks * (kBlock / 64);
    int per_wave = (count + target_waves - 1) / target_waves;
    if (per_wave < 1) per_wave = 1;
    if (per_wave > 64) per_wave = 64;
    const int waves = (count + per_wave - 1) / per_wave;
    int blocks = (waves + 3) / 4;
    if (blocks > max_blocks) blocks = max_blocks;
    hipLaunchKernelGGL(zc_gather_sg<4>, dim3(blocks), dim3(kBlock), 0, st, entries, count, per_wave);
    return (int)hipGetLastError();
}
