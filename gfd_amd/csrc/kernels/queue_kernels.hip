// GFD Queue mode kernels: GPU-submitted descriptors and a bounded completion
// wait (the reference's examples/04_benchmark.cu:31-54 bench_gfd_submit_kernel
// / bench_gfd_wait_kernel, on the wave64 device API of include/gfd/device.h).
#include <hip/hip_runtime.h>

#include <cstring>

#include "gfd/device.h"
#include "gfd_capi.h"

namespace {

// One lane per descriptor.
__global__ __launch_bounds__(256) void queue_submit_tokens_kernel(gfd::DescriptorQueue* queue,
                                                                  const gfd::TokenInfo* __restrict__ tokens,
                                                                  void* gpu_dst, int num_tokens,
                                                                  uint32_t token_size, uint64_t base_slot) {
    const int tid = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    const bool active = tid < num_tokens;
    gfd::device::write_and_commit(queue, base_slot, tid, active, active ? tokens[tid].cpu_addr : 0, gpu_dst,
                                  token_size, num_tokens);
}

// Backpressure form (the reference's write_descriptor_safe, device.cuh:120-152,
// with the caller's retry it asks for): lane j writes descriptor j at slot
// base_slot + j only once the poller has consumed that slot, retrying with
// s_sleep; the wait is bounded by max_ticks (then *status = 1 and the lane
// gives up).  Launches may hold more descriptors than QUEUE_SIZE: lanes of a
// later lap wait for the earlier lap's slots, which lower-numbered
// workgroups (dispatched first, never waiting themselves) have committed.
// full_count (HBM, optional) counts lanes that found their slot occupied.
__global__ __launch_bounds__(256) void queue_submit_safe_kernel(gfd::DescriptorQueue* queue,
                                                                const gfd::TokenInfo* __restrict__ tokens,
                                                                void* gpu_dst, int num_tokens, uint32_t token_size,
                                                                uint64_t base_slot, uint64_t max_ticks, int* status,
                                                                unsigned int* full_count) {
    const int tid = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (tid >= num_tokens) return;
    const uint64_t src = tokens[tid].cpu_addr;
    const uint64_t t0 = wall_clock64();
    bool waited = false;
    while (!gfd::device::write_descriptor_safe(queue, base_slot, tid, src, gpu_dst, token_size, num_tokens)) {
        waited = true;
        if (wall_clock64() - t0 > max_ticks) {
            __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return;
        }
        __builtin_amdgcn_s_sleep(8);
    }
    gfd::device::commit_slot(queue, base_slot + (uint64_t)tid);
    if (waited && full_count) atomicAdd(full_count, 1u);
}

__global__ void queue_wait_kernel(gfd::DescriptorQueue* queue, uint64_t expected_done, uint64_t max_ticks,
                                  int* status) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        const bool ok = gfd::device::wait_for_completion(queue, expected_done, max_ticks);
        __hip_atomic_store(status, ok ? 0 : 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// Fused request + wait + consume in one launch (the reference's
// examples/01_basic_transfer.cu:27-85 fused_prefetch_and_compute_kernel):
// every lane writes and commits its token's descriptor; lane 0 of each
// workgroup waits (bounded) until the poller has landed all of them; then the
// workgroup's waves read their tokens from HBM and write each token's u32-word
// checksum (an integer sum, so the result is exact).  Every workgroup of the
// launch must be resident at once (it waits for descriptors the others
// write): num_tokens <= QUEUE_SIZE keeps the grid at 64 workgroups.
__global__ __launch_bounds__(256) void queue_fused_checksum_kernel(gfd::DescriptorQueue* queue,
                                                                   const gfd::TokenInfo* __restrict__ tokens,
                                                                   void* gpu_dst, int num_tokens, uint32_t token_size,
                                                                   uint64_t base_slot, uint64_t max_ticks,
                                                                   unsigned long long* __restrict__ sums,
                                                                   int* status) {
    __shared__ int landed;
    const int tid = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    const bool active = tid < num_tokens;
    if (active)
        gfd::device::write_descriptor(queue, base_slot, tid, tokens[tid].cpu_addr, gpu_dst, token_size, num_tokens);
    gfd::device::fence_and_commit(queue, base_slot, tid, active);
    if (threadIdx.x == 0)
        landed = gfd::device::wait_for_completion(queue, base_slot + (uint64_t)num_tokens, max_ticks) ? 1 : 0;
    __syncthreads();
    if (!landed) {
        if (threadIdx.x == 0) __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return;
    }
    // The copy engines wrote the tokens: every lane acquires before reading.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
    const int lane = (int)(threadIdx.x & 63), wave = (int)(threadIdx.x >> 6), nwaves = (int)(blockDim.x >> 6);
    const int first = (int)(blockIdx.x * blockDim.x), last = min(num_tokens, first + (int)blockDim.x);
    const uint32_t nw = token_size / 4;
    for (int j = first + wave; j < last; j += nwaves) {
        const uint8_t* p = (const uint8_t*)gpu_dst + (uint64_t)j * token_size;
        unsigned long long acc = 0;
        if (((uintptr_t)p & 3) == 0) {
            const uint32_t* w = (const uint32_t*)p;
            for (uint32_t k = (uint32_t)lane; k < nw; k += 64) acc += w[k];
        } else {
            for (uint32_t k = (uint32_t)lane; k < nw; k += 64)
                acc += (uint32_t)p[4 * k] | ((uint32_t)p[4 * k + 1] << 8) | ((uint32_t)p[4 * k + 2] << 16) |
                       ((uint32_t)p[4 * k + 3] << 24);
        }
        for (uint32_t b = nw * 4 + (uint32_t)lane; b < token_size; b += 64) acc += p[b];
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)acc, o, 64);
            const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(acc >> 32), o, 64);
            acc += ((unsigned long long)hi << 32) | lo;
        }
        if (lane == 0) sums[j] = acc;
    }
}

}  // namespace

extern "C" int gfd_queue_alloc(void** queue) {
    if (!queue) return (int)hipErrorInvalidValue;
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, sizeof(gfd::DescriptorQueue), hipHostMallocCoherent);
    if (e != hipSuccess) return (int)e;
    std::memset(p, 0, sizeof(gfd::DescriptorQueue));
    *queue = p;
    return 0;
}

extern "C" int gfd_queue_free(void* queue) { return queue ? (int)hipHostFree(queue) : 0; }

extern "C" int gfd_queue_submit_tokens(void* queue, const void* tokens, void* gpu_dst, int num_tokens,
                                       uint32_t token_size, uint64_t base_slot, void* stream) {
    if (!queue || num_tokens < 0 || (num_tokens > 0 && (!tokens || !gpu_dst || token_size == 0)))
        return (int)hipErrorInvalidValue;
    if (num_tokens == 0) return 0;
    auto* q = (gfd::DescriptorQueue*)queue;
    // The ring must have room: slots [base_slot, base_slot + n) may not lap
    // slots the poller has not consumed yet.
    const uint64_t read = __atomic_load_n(&q->read_idx, __ATOMIC_ACQUIRE);
    if (num_tokens > gfd::QUEUE_SIZE || base_slot < read || base_slot + (uint64_t)num_tokens - read > (uint64_t)gfd::QUEUE_SIZE)
        return (int)hipErrorInvalidValue;
    const int threads = 256;
    const int blocks = (num_tokens + threads - 1) / threads;
    hipLaunchKernelGGL(queue_submit_tokens_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)stream, q,
                       (const gfd::TokenInfo*)tokens, gpu_dst, num_tokens, token_size, base_slot);
    return (int)hipGetLastError();
}

extern "C" int gfd_queue_submit_tokens_safe(void* queue, const void* tokens, void* gpu_dst, int num_tokens,
                                            uint32_t token_size, uint64_t base_slot, uint64_t timeout_us, int* status,
                                            unsigned int* full_count, void* stream) {
    if (!queue || !status || num_tokens < 0 || (num_tokens > 0 && (!tokens || !gpu_dst || token_size == 0)))
        return (int)hipErrorInvalidValue;
    if (num_tokens == 0) return 0;
    auto* q = (gfd::DescriptorQueue*)queue;
    if (base_slot < __atomic_load_n(&q->read_idx, __ATOMIC_ACQUIRE)) return (int)hipErrorInvalidValue;
    const uint64_t ticks = timeout_us * (gfd::device::kWallClockHz / 1000000ull);
    const int threads = 256;
    const int blocks = (num_tokens + threads - 1) / threads;
    hipLaunchKernelGGL(queue_submit_safe_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)stream, q,
                       (const gfd::TokenInfo*)tokens, gpu_dst, num_tokens, token_size, base_slot, ticks, status,
                       full_count);
    return (int)hipGetLastError();
}

extern "C" int gfd_queue_fused_checksums(void* queue, const void* tokens, void* gpu_dst, int num_tokens,
                                         uint32_t token_size, uint64_t base_slot, uint64_t timeout_us,
                                         unsigned long long* sums, int* status, void* stream) {
    if (!queue || !status || !sums || num_tokens <= 0 || !tokens || !gpu_dst || token_size == 0)
        return (int)hipErrorInvalidValue;
    auto* q = (gfd::DescriptorQueue*)queue;
    const uint64_t read = __atomic_load_n(&q->read_idx, __ATOMIC_ACQUIRE);
    if (num_tokens > gfd::QUEUE_SIZE || base_slot < read || base_slot + (uint64_t)num_tokens - read > (uint64_t)gfd::QUEUE_SIZE)
        return (int)hipErrorInvalidValue;
    const uint64_t ticks = timeout_us * (gfd::device::kWallClockHz / 1000000ull);
    const int threads = 256;
    const int blocks = (num_tokens + threads - 1) / threads;
    hipLaunchKernelGGL(queue_fused_checksum_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)stream, q,
                       (const gfd::TokenInfo*)tokens, gpu_dst, num_tokens, token_size, base_slot, ticks, sums, status);
    return (int)hipGetLastError();
}

extern "C" int gfd_queue_wait(void* queue, uint64_t expected_done, uint64_t timeout_us, int* status,
                              void* stream) {
    if (!queue || !status) return (int)hipErrorInvalidValue;
    const uint64_t ticks = timeout_us * (gfd::device::kWallClockHz / 1000000ull);
    hipLaunchKernelGGL(queue_wait_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (gfd::DescriptorQueue*)queue,
                       expected_done, ticks, status);
    return (int)hipGetLastError();
}
