// GPU-side dynamic SG list submission, written the way the reference's
// test/test_sg_gpu_submit.cu is: the caller writes its own combined kernel
// (transfer, compute and submitter waves), launches it with
// hipLaunchKernelGGL on the session's queues, brackets it with
// session.get_poller()->start() / hipDeviceSynchronize() /
// session.get_poller()->stop(), and checks the floats i + 1 of every entry.
//
// MI355X form of the kernel: waves of 64 lanes; the transfer and compute
// waves are the library's SG transfer loop (waves 0 and 1), which copies each
// committed list itself; wave 2 submits the lists with the sg:: primitives
// and, once every list has landed, ends the launch.
//
// Three rounds on one session: two caller-launched kernels (the second
// starts on the state the poller's stop() leaves) and one through
// session.launch(), whose counts then show in the poller's stats as well.
// Prints PASSED and exits 0 on success.
#include <gfd/gfd.h>
#include <gfd/sg_device_primitives.cuh>
#include <gfd/sg_warp_spec.cuh>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <vector>

#define HIP_OK(call)                                                               \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) {                                                    \
            std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_)); \
            return 1;                                                              \
        }                                                                          \
    } while (0)

struct NullCompute {
    __device__ void operator()(gfd::sg_warp_spec::SGListView) const {}
};
GFD_SG_WARP_SPEC_KERNEL(sg_null_kernel, NullCompute);

// Wave 0: transfer, wave 1: compute, wave 2: submitter.
__global__ __launch_bounds__(192) void gpu_submit_test_kernel(gfd::DescriptorQueue* dq, gfd::SGTaskQueue* sq,
                                                              NullCompute compute_fn, const float* cpu_base,
                                                              float* gpu_base, int entries_per_list, int num_lists,
                                                              uint32_t entry_size) {
    gfd::sg_warp_spec::_sg_transfer_warp_loop(dq, sq, compute_fn);  // waves 0 and 1; wave 2 returns
    if (gfd::wave::wave_id() != 2) return;
    const int lane = gfd::wave::lane_id();
    for (int list = 0; list < num_lists; list++) {
        if (!gfd::sg::sg_wait_entry_space(sq, (uint32_t)entries_per_list)) return;
        const uint64_t pool_offset = gfd::sg::sg_alloc_entries(sq, (uint32_t)entries_per_list);
        for (int i = lane; i < entries_per_list; i += 64) {
            gfd::DeviceSGEntry& e = sq->entries[(pool_offset + (uint64_t)i) % gfd::MAX_SG_POOL_ENTRIES];
            const uint64_t g = (uint64_t)list * (uint64_t)entries_per_list + (uint64_t)i;
            e.src_addr = (uint64_t)(uintptr_t)cpu_base + g * entry_size;
            e.dst_addr = (uint64_t)(uintptr_t)gpu_base + g * entry_size;
            e.size = entry_size;
            e.tag = (uint32_t)list;
        }
        if (!gfd::sg::sg_wait_list_space(sq)) return;
        const uint64_t slot = gfd::sg::sg_alloc_list(sq);
        if (!gfd::sg::sg_commit_list(sq, slot, (uint32_t)pool_offset, (uint32_t)entries_per_list, (uint32_t)list,
                                     gfd::SG_FLAG_NONE))
            return;
    }
    // Every list landed: nothing is left to copy, so the transfer waves stop.
    if (gfd::sg::sg_wait_gpu_lists_done(sq, (uint64_t)num_lists))
        gfd::sg::sg_terminate_all_landed(sq);
    else
        gfd::sg::sg_terminate(sq);
}

// The per-poller summary of the reference's examples/07_warp_spec_simple.cu.
static void print_poller_stats(gfd::CpuPollingThread& poller, double elapsed_ms) {
    const uint64_t descs = poller.get_descriptors_processed();
    const double bytes = poller.get_total_bytes_copied();
    std::printf("    [Poller] descs=%llu, batches=%llu, coalesced=%llu\n", (unsigned long long)descs,
                (unsigned long long)poller.get_batches_submitted(), (unsigned long long)poller.get_coalesced_entries());
    std::printf("    [Poller] bytes=%.2f MB, gather=%llu us, submit=%llu us, wait=%llu us\n", bytes / (1024.0 * 1024.0),
                (unsigned long long)poller.get_gather_us(), (unsigned long long)poller.get_dma_submit_us(),
                (unsigned long long)poller.get_dma_wait_us());
    if (elapsed_ms > 0 && descs > 0)
        std::printf("    [Poller] effective BW=%.2f GB/s, descs/ms=%.0f\n", bytes / (elapsed_ms * 1e6),
                    (double)descs / elapsed_ms);
}

static int check(const float* cpu, float* gpu, size_t n, const char* what) {
    std::vector<float> h(n);
    if (hipMemcpy(h.data(), gpu, n * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) return -1;
    int errors = 0;
    for (size_t i = 0; i < n; i++)
        if (std::fabs(cpu[i] - h[i]) > 1e-5f && errors++ < 3)
            std::fprintf(stderr, "  %s: mismatch at %zu: expected %.1f got %.1f\n", what, i, cpu[i], h[i]);
    std::printf("  %s data correctness: %s (%d errors)\n", what, errors == 0 ? "PASS" : "FAIL", errors);
    return errors;
}

int main() {
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    if (hipSetDevice(0) != hipSuccess) return 1;
    constexpr int NUM_LISTS = 4;
    constexpr int ENTRIES_PER_LIST = 8;
    constexpr int TOTAL_ENTRIES = NUM_LISTS * ENTRIES_PER_LIST;
    constexpr uint32_t ENTRY_SIZE = 4096;
    constexpr size_t TOTAL_SIZE = (size_t)TOTAL_ENTRIES * ENTRY_SIZE;
    constexpr size_t N = TOTAL_SIZE / sizeof(float);

    float* cpu_data = nullptr;
    HIP_OK(hipHostMalloc((void**)&cpu_data, TOTAL_SIZE, hipHostMallocDefault));
    for (size_t i = 0; i < N; i++) cpu_data[i] = (float)(i + 1);
    float* gpu_data = nullptr;
    HIP_OK(hipMalloc((void**)&gpu_data, TOTAL_SIZE));

    gfd::SGWarpSpecConfig config;
    config.num_compute_warps = 1;
    config.num_blocks = 1;
    config.use_copy_engine = true;
    config.idle_limit_ms = 10000;
    bool ok = true;
    {
        gfd::SGWarpSpecSession session(config);
        for (int round = 0; round < 2; round++) {
            HIP_OK(hipMemset(gpu_data, 0, TOTAL_SIZE));
            HIP_OK(hipDeviceSynchronize());
            std::printf("round %d: launching the 3-wave kernel (%d lists x %d entries)\n", round, NUM_LISTS,
                        ENTRIES_PER_LIST);
            hipLaunchKernelGGL(gpu_submit_test_kernel, dim3(1), dim3(192), 0, 0, session.get_desc_queue(),
                               session.get_sg_queue(), NullCompute{}, cpu_data, gpu_data, ENTRIES_PER_LIST,
                               NUM_LISTS, ENTRY_SIZE);
            HIP_OK(hipGetLastError());
            session.get_poller()->start();
            HIP_OK(hipDeviceSynchronize());
            session.get_poller()->stop();
            const auto stats = session.get_stats();
            std::printf("  Poller: desc=%llu bytes=%.2f MB, session errors 0x%llx\n",
                        (unsigned long long)stats.descriptors_processed, stats.bytes_transferred / (1024.0 * 1024.0),
                        (unsigned long long)session.error_bits());
            if (stats.descriptors_processed != TOTAL_ENTRIES || stats.bytes_transferred != TOTAL_SIZE ||
                session.lists_landed() != NUM_LISTS || session.error_bits() != 0)
                ok = false;
            if (check(cpu_data, gpu_data, N, round == 0 ? "raw launch 1" : "raw launch 2") != 0) ok = false;
        }
        // The poller's stats count what the transfer waves landed.
        gfd::CpuPollingThread* poller = session.get_poller();
        print_poller_stats(*poller, 0.0);
        if (poller->get_descriptors_processed() != 2u * TOTAL_ENTRIES ||
            poller->get_total_bytes_copied() != 2.0 * (double)TOTAL_SIZE || poller->get_batches_submitted() != 2u * NUM_LISTS) {
            std::fprintf(stderr, "  poller stats do not count the two launches\n");
            ok = false;
        }
        // Then a host-submitted round through the session's own launch path.
        HIP_OK(hipMemset(gpu_data, 0, TOTAL_SIZE));
        HIP_OK(hipDeviceSynchronize());
        std::vector<gfd::DeviceSGEntry> e(TOTAL_ENTRIES);
        for (int i = 0; i < TOTAL_ENTRIES; i++)
            e[i] = gfd::DeviceSGEntry{(uint64_t)(uintptr_t)cpu_data + (uint64_t)i * ENTRY_SIZE,
                                      (uint64_t)(uintptr_t)gpu_data + (uint64_t)i * ENTRY_SIZE, ENTRY_SIZE, 0};
        if (session.submit_sg_list(e.data(), TOTAL_ENTRIES, 0) == ~0ull) ok = false;
        session.launch(sg_null_kernel, NullCompute{});
        if (!session.synchronize()) ok = false;
        if (check(cpu_data, gpu_data, N, "session launch") != 0) ok = false;
        print_poller_stats(*poller, session.get_stats().elapsed_ms);
        if (poller->get_descriptors_processed() != 3u * TOTAL_ENTRIES) ok = false;
    }
    HIP_OK(hipFree(gpu_data));
    HIP_OK(hipHostFree(cpu_data));
    std::printf("  Verify:    %s\n", ok ? "PASSED" : "FAILED");
    return ok ? 0 : 1;
}
