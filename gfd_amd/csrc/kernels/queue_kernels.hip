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

__global__ void queue_wait_kernel(gfd::DescriptorQueue* queue, uint64_t expected_done, uint64_t max_ticks,
                                  int* status) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        const bool ok = gfd::device::wait_for_completion(queue, expected_done, max_ticks);
        __hip_atomic_store(status, ok ? 0 : 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
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

extern "C" int gfd_queue_wait(void* queue, uint64_t expected_done, uint64_t timeout_us, int* status,
                              void* stream) {
    if (!queue || !status) return (int)hipErrorInvalidValue;
    const uint64_t ticks = timeout_us * (gfd::device::kWallClockHz / 1000000ull);
    hipLaunchKernelGGL(queue_wait_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (gfd::DescriptorQueue*)queue,
                       expected_done, ticks, status);
    return (int)hipGetLastError();
}
