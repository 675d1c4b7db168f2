// Device code written the way the reference's tests are
// (test/test_sg_e2e.cu and test/test_db_small_tiles.cu of the reference): it
// includes <gfd/gfd.h> and the device headers by their reference names
// (<gfd/sg_warp_spec.cuh>, <gfd/warp_spec.cuh>), generates its kernels with
// GFD_SG_WARP_SPEC_KERNEL and GFD_WARP_SPEC_KERNEL_DB around its own
// functors, and runs them through SGWarpSpecSession and WarpSpecSession.
// Runtime calls are the HIP API where the reference calls the CUDA runtime.
//
// Known answers as in the reference: the SG list lands floats i + 1 (every
// one compared); the double-buffered tiles give per-token sums (t + 1) * dim
// for tile counts 1, 2, 3, 4, 5 and 7 (test_db_small_tiles' cases).  The
// functors stride over 64-lane waves.  Prints PASSED and exits 0 on success.
#include <gfd/gfd.h>
#include <gfd/sg_warp_spec.cuh>
#include <gfd/warp_spec.cuh>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <vector>

#define HIP_OK(call)                                                                  \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) {                                                       \
            std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));    \
            return false;                                                             \
        }                                                                             \
    } while (0)

// Counts the landed lists' entries (the reference's NullCompute prints them).
struct CountCompute {
    unsigned int* seen;
    __device__ void operator()(gfd::sg_warp_spec::SGListView list) {
        if (list.lane_id == 0) atomicAdd(seen, list.count);
    }
};
GFD_SG_WARP_SPEC_KERNEL(sg_test_kernel, CountCompute);

struct SimpleReduce {
    float* output;
    int token_dim;
    __device__ void operator()(gfd::warp_spec::ChunkView chunk) {
        for (uint32_t i = (uint32_t)chunk.lane_id; i < chunk.size; i += 64) {
            const float* token = chunk.data<float>((int)i);
            float sum = 0.0f;
            for (int d = 0; d < token_dim; d++) sum += token[d];
            output[chunk.global_idx((int)i)] = sum;
        }
    }
};
GFD_WARP_SPEC_KERNEL_DB(test_kernel_db, SimpleReduce);

static bool sg_e2e() {
    constexpr int N = 4;
    constexpr size_t TOKEN_SIZE = 4096;
    constexpr size_t TOTAL = N * TOKEN_SIZE;
    float* cpu_data = nullptr;
    HIP_OK(hipHostMalloc((void**)&cpu_data, TOTAL, hipHostMallocDefault));
    for (size_t i = 0; i < TOTAL / sizeof(float); i++) cpu_data[i] = (float)(i + 1);
    float* gpu_data = nullptr;
    HIP_OK(hipMalloc((void**)&gpu_data, TOTAL));
    HIP_OK(hipMemset(gpu_data, 0, TOTAL));
    unsigned int* seen = nullptr;
    HIP_OK(hipMalloc((void**)&seen, sizeof(unsigned int)));
    HIP_OK(hipMemset(seen, 0, sizeof(unsigned int)));
    HIP_OK(hipDeviceSynchronize());

    gfd::SGWarpSpecConfig config;
    config.num_compute_warps = 1;
    config.num_blocks = 1;
    config.use_copy_engine = true;
    config.idle_limit_ms = 10000;
    bool ok = true;
    {
        gfd::SGWarpSpecSession session(config);
        gfd::DeviceSGEntry entries[N];
        for (int i = 0; i < N; i++) {
            entries[i].src_addr = (uint64_t)(uintptr_t)cpu_data + (uint64_t)i * TOKEN_SIZE;
            entries[i].dst_addr = (uint64_t)(uintptr_t)gpu_data + (uint64_t)i * TOKEN_SIZE;
            entries[i].size = TOKEN_SIZE;
            entries[i].tag = 0;
        }
        if (session.submit_sg_list(entries, N, 0, gfd::SG_FLAG_HOST_SUBMITTED) == ~0ull) ok = false;
        session.launch(sg_test_kernel, CountCompute{seen});
        if (!session.synchronize()) ok = false;
        const auto stats = session.get_stats();
        std::printf("SG session: %llu entries, %llu bytes, %.3f ms\n", (unsigned long long)stats.descriptors_processed,
                    (unsigned long long)stats.bytes_transferred, stats.elapsed_ms);
        if (stats.descriptors_processed != N || stats.bytes_transferred != TOTAL) ok = false;
    }
    std::vector<float> h(TOTAL / sizeof(float));
    unsigned int h_seen = 0;
    HIP_OK(hipMemcpy(h.data(), gpu_data, TOTAL, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(&h_seen, seen, sizeof(h_seen), hipMemcpyDeviceToHost));
    int errors = 0;
    for (size_t i = 0; i < h.size(); i++)
        if (h[i] != cpu_data[i] && errors++ < 3) std::fprintf(stderr, "  Mismatch at %zu: %.1f vs %.1f\n", i, h[i], cpu_data[i]);
    if (h_seen != N) {
        std::fprintf(stderr, "  compute functor saw %u entries, expected %d\n", h_seen, N);
        ok = false;
    }
    std::printf("SG data: %s (%d errors)\n", errors == 0 ? "PASS" : "FAIL", errors);
    HIP_OK(hipFree(seen));
    HIP_OK(hipFree(gpu_data));
    HIP_OK(hipHostFree(cpu_data));
    return ok && errors == 0;
}

static bool db_tiles(int total_tokens, int tokens_per_tile, int tokens_per_chunk, int token_dim, int num_cus) {
    const int num_tiles = total_tokens / tokens_per_tile;
    const size_t token_size = (size_t)token_dim * sizeof(float);
    const size_t total_size = (size_t)total_tokens * token_size;
    float* cpu_data = nullptr;
    HIP_OK(hipHostMalloc((void**)&cpu_data, total_size, hipHostMallocDefault));
    for (int t = 0; t < total_tokens; t++)
        for (int d = 0; d < token_dim; d++) cpu_data[(size_t)t * token_dim + d] = (float)(t + 1);
    float *gpu_data = nullptr, *d_output = nullptr;
    HIP_OK(hipMalloc((void**)&gpu_data, total_size));
    HIP_OK(hipMalloc((void**)&d_output, (size_t)total_tokens * sizeof(float)));
    HIP_OK(hipMemset(gpu_data, 0, total_size));
    HIP_OK(hipMemset(d_output, 0, (size_t)total_tokens * sizeof(float)));
    HIP_OK(hipDeviceSynchronize());

    gfd::WarpSpecConfig config;
    config.total_tokens = (uint32_t)total_tokens;
    config.token_size = (uint32_t)token_size;
    config.cpu_src = cpu_data;
    config.gpu_dst = gpu_data;
    config.tokens_per_tile = (uint32_t)tokens_per_tile;
    config.tokens_per_chunk = (uint32_t)tokens_per_chunk;
    config.num_blocks = num_cus < num_tiles ? num_cus : num_tiles;
    config.double_buffer = true;
    bool ok = true;
    {
        gfd::WarpSpecSession session(config);
        session.launch(test_kernel_db, SimpleReduce{d_output, token_dim});
        ok = session.synchronize();
    }
    std::vector<float> h((size_t)total_tokens);
    HIP_OK(hipMemcpy(h.data(), d_output, h.size() * sizeof(float), hipMemcpyDeviceToHost));
    int errors = 0;
    for (int t = 0; t < total_tokens; t++) {
        const float expected = (float)(t + 1) * (float)token_dim;
        if (!std::isfinite(h[(size_t)t]) || std::fabs(h[(size_t)t] - expected) > 1.0f) errors++;
    }
    std::printf("  tiles=%d tokens=%d tile=%d chunk=%d: %s\n", num_tiles, total_tokens, tokens_per_tile,
                tokens_per_chunk, ok && errors == 0 ? "PASS" : "FAIL");
    HIP_OK(hipFree(d_output));
    HIP_OK(hipFree(gpu_data));
    HIP_OK(hipHostFree(cpu_data));
    return ok && errors == 0;
}

int main() {
    if (hipSetDevice(0) != hipSuccess) return 1;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess) return 1;
    bool ok = sg_e2e();
    for (int tiles : {1, 2, 3, 4, 5, 7}) ok = db_tiles(tiles * 64, 64, 16, 128, cus) && ok;
    std::printf("  Verify:    %s\n", ok ? "PASSED" : "FAILED");
    return ok ? 0 : 1;
}
