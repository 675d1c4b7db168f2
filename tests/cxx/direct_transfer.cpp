// A host program written the way the reference's callers are
// (examples/02_direct_transfer.cu of the reference): it includes <gfd/gfd.h>,
// pre-allocates the StagingPool, creates a CpuPollingThread with the direct
// copy channels, starts it, and gathers 1024 tokens of 4 KiB scattered at 2x
// stride with submit_direct.  The runtime calls are the HIP host API
// (hipHostMalloc, hipMalloc, hipMemcpy) where the reference calls the CUDA
// runtime; every gfd:: call is the reference's.
//
// Known-answer check as in the reference: token i is filled with i & 0xFF and
// every byte of the destination is compared.  Then the same tokens in a
// seeded random order, and a check that the poller took its Queue staging
// from the pool.  Prints PASSED and exits 0 on success.
#include <gfd/gfd.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#define HIP_OK(call)                                                                  \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) {                                                       \
            std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));    \
            return 1;                                                                 \
        }                                                                             \
    } while (0)

static int check(const uint8_t* got, const std::vector<int>& order, int n, size_t T) {
    for (int j = 0; j < n; j++) {
        const uint8_t want = (uint8_t)(order[j] & 0xFF);
        for (size_t b = 0; b < T; b++)
            if (got[(size_t)j * T + b] != want) {
                std::fprintf(stderr, "MISMATCH at token %d, byte %zu: got 0x%02X, expected 0x%02X\n", j, b,
                             got[(size_t)j * T + b], want);
                return 1;
            }
    }
    return 0;
}

int main() {
    constexpr int NUM_TOKENS = 1024;
    constexpr size_t TOKEN_SIZE = 4096;
    constexpr size_t TOTAL_SIZE = (size_t)NUM_TOKENS * TOKEN_SIZE;
    constexpr int SCATTER_STRIDE = 2;

    HIP_OK(hipSetDevice(0));
    gfd::TopologyConfig topo = gfd::discover_topology(1);
    gfd::print_topology(topo);

    char* cpu_buf = nullptr;
    HIP_OK(hipHostMalloc((void**)&cpu_buf, TOTAL_SIZE * SCATTER_STRIDE, hipHostMallocDefault));
    for (int i = 0; i < NUM_TOKENS; i++)
        std::memset(cpu_buf + (size_t)i * TOKEN_SIZE * SCATTER_STRIDE, (uint8_t)(i & 0xFF), TOKEN_SIZE);
    char* gpu_buf = nullptr;
    HIP_OK(hipMalloc((void**)&gpu_buf, TOTAL_SIZE));
    HIP_OK(hipMemset(gpu_buf, 0, TOTAL_SIZE));
    HIP_OK(hipDeviceSynchronize());

    // Descriptor queue (needed by the poller, unused by Direct): fine-grained host memory.
    gfd::DescriptorQueue* queue = nullptr;
    HIP_OK(hipHostMalloc((void**)&queue, sizeof(gfd::DescriptorQueue), hipHostMallocCoherent));
    std::memset(queue, 0, sizeof(gfd::DescriptorQueue));

    if (!gfd::StagingPool::instance().init(1, TOTAL_SIZE)) {
        std::fprintf(stderr, "StagingPool init failed\n");
        return 1;
    }
    int rc = 0;
    {
        gfd::CpuPollingThread poller(queue, gpu_buf, cpu_buf, TOTAL_SIZE, /*use_ce=*/true, /*numa_node=*/0,
                                     /*core_offset=*/0, /*num_ce_channels=*/0, /*exclusive_core_base=*/0,
                                     /*exclusive_core_count=*/32);
        if (!poller.init_copy_engine()) {
            std::fprintf(stderr, "Failed to init copy engine\n");
            return 1;
        }
        poller.init_direct_ce();
        poller.start();
        if (poller.staging_pool_set() < 0 || !poller.is_running()) {
            std::fprintf(stderr, "poller did not take a pool set (%d) or is not running\n", poller.staging_pool_set());
            rc = 1;
        }

        gfd::SGEntry* entries = new gfd::SGEntry[NUM_TOKENS];
        std::vector<int> order(NUM_TOKENS);
        std::vector<uint8_t> verify(TOTAL_SIZE);
        for (int pass = 0; pass < 2 && rc == 0; pass++) {
            for (int i = 0; i < NUM_TOKENS; i++) order[i] = i;
            if (pass == 1) {  // seeded Fisher-Yates order (xorshift64)
                uint64_t s = 0xD1B54A32D192ED03ull;
                for (int i = NUM_TOKENS - 1; i > 0; i--) {
                    s ^= s << 13;
                    s ^= s >> 7;
                    s ^= s << 17;
                    std::swap(order[i], order[(int)(s % (uint64_t)(i + 1))]);
                }
            }
            for (int j = 0; j < NUM_TOKENS; j++) {
                entries[j].dst = (gfd::DevicePtr)(gpu_buf + (size_t)j * TOKEN_SIZE);
                entries[j].src = cpu_buf + (size_t)order[j] * TOKEN_SIZE * SCATTER_STRIDE;
                entries[j].size = TOKEN_SIZE;
            }
            HIP_OK(hipMemset(gpu_buf, 0, TOTAL_SIZE));
            HIP_OK(hipDeviceSynchronize());
            for (int i = 0; i < 10; i++)
                if (poller.submit_direct(entries, NUM_TOKENS) < 0) rc = 1;
            const double us = poller.submit_direct(entries, NUM_TOKENS);
            if (us < 0) rc = 1;
            std::printf("%s order: %.1f us, %.2f GB/s\n", pass ? "random" : "in", us, TOTAL_SIZE / (us * 1e3));
            HIP_OK(hipMemcpy(verify.data(), gpu_buf, TOTAL_SIZE, hipMemcpyDeviceToHost));
            if (rc == 0) rc = check(verify.data(), order, NUM_TOKENS, TOKEN_SIZE);
        }
        delete[] entries;
        poller.stop();
    }
    gfd::StagingPool::instance().shutdown();
    std::printf("  Verify:    %s\n", rc == 0 ? "PASSED" : "FAILED");
    HIP_OK(hipFree(gpu_buf));
    HIP_OK(hipHostFree(queue));
    HIP_OK(hipHostFree(cpu_buf));
    return rc;
}
