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
// functors stride over 64-lane waves.  Added: eight lists on a session with
// three compute waves, where a functor declaring kSharesLists has each list
// split between the three and one without it sees each list once; every
// entry must be marked exactly once either way.  After each tile case the
// session poller's stats are printed as examples/07_warp_spec_simple.cu:283
// does, and must count the tokens the launch landed.  Prints PASSED and
// exits 0 on success.
#include <gfd/gfd.h>
#include <gfd/sg_warp_spec.cuh>
#include <gfd/warp_spec.cuh>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
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

// Marks every entry it is given (by tag) once.  With kSharesLists the
// session's compute waves share each list: wave `part` takes entries part,
// part + parts, ...
struct SharedTouch {
    static constexpr bool kSharesLists = true;
    unsigned int* touched;
    unsigned int* parts_seen;
    __device__ void operator()(gfd::sg_warp_spec::SGListView list) {
        if (list.lane_id == 0) atomicMax(parts_seen, list.parts);
        for (uint32_t i = list.part + (uint32_t)list.lane_id * list.parts; i < list.count; i += 64u * list.parts)
            atomicAdd(&touched[list.get_entry(i).tag], 1u);
    }
};
GFD_SG_WARP_SPEC_KERNEL(sg_shared_kernel, SharedTouch);

// The same marking without kSharesLists: one compute wave per list, however
// many the session has.
struct SoloTouch {
    unsigned int* touched;
    unsigned int* parts_seen;
    __device__ void operator()(gfd::sg_warp_spec::SGListView list) {
        if (list.lane_id == 0) atomicMax(parts_seen, list.parts);
        for (uint32_t i = (uint32_t)list.lane_id; i < list.count; i += 64u)
            atomicAdd(&touched[list.get_entry(i).tag], 1u);
    }
};
GFD_SG_WARP_SPEC_KERNEL(sg_solo_kernel, SoloTouch);

// 8 lists of 100 entries, 3 compute waves per workgroup: every entry must be
// marked exactly once, by 3 sharing waves or by wave 1 alone.
template <typename Functor, typename Kernel>
static bool sg_compute_waves(Kernel kernel, unsigned int want_parts, const char* name) {
    constexpr int LISTS = 8, PER = 100, N = LISTS * PER;
    constexpr size_t TOKEN = 1024;
    char* cpu_data = nullptr;
    HIP_OK(hipHostMalloc((void**)&cpu_data, (size_t)N * TOKEN, hipHostMallocDefault));
    for (size_t i = 0; i < (size_t)N * TOKEN; i++) cpu_data[i] = (char)(i * 7 + 3);
    char* gpu_data = nullptr;
    unsigned int *touched = nullptr, *parts_seen = nullptr;
    HIP_OK(hipMalloc((void**)&gpu_data, (size_t)N * TOKEN));
    HIP_OK(hipMalloc((void**)&touched, N * sizeof(unsigned int)));
    HIP_OK(hipMalloc((void**)&parts_seen, sizeof(unsigned int)));
    HIP_OK(hipMemset(touched, 0, N * sizeof(unsigned int)));
    HIP_OK(hipMemset(parts_seen, 0, sizeof(unsigned int)));
    HIP_OK(hipDeviceSynchronize());
    gfd::SGWarpSpecConfig config;
    config.num_compute_warps = 3;
    config.num_blocks = 4;
    config.idle_limit_ms = 10000;
    bool ok = true;
    {
        gfd::SGWarpSpecSession session(config);
        std::vector<gfd::DeviceSGEntry> e(PER);
        for (int l = 0; l < LISTS; l++) {
            for (int i = 0; i < PER; i++) {
                const int k = l * PER + i;
                e[i].src_addr = (uint64_t)(uintptr_t)cpu_data + (uint64_t)k * TOKEN;
                e[i].dst_addr = (uint64_t)(uintptr_t)gpu_data + (uint64_t)k * TOKEN;
                e[i].size = TOKEN;
                e[i].tag = (uint32_t)k;
            }
            if (session.submit_sg_list(e.data(), PER, (uint32_t)l, gfd::SG_FLAG_HOST_SUBMITTED) == ~0ull) ok = false;
        }
        session.launch(kernel, Functor{touched, parts_seen});
        if (!session.synchronize()) ok = false;
    }
    std::vector<unsigned int> h(N);
    std::vector<char> landed((size_t)N * TOKEN);
    unsigned int h_parts = 0;
    HIP_OK(hipMemcpy(h.data(), touched, N * sizeof(unsigned int), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(&h_parts, parts_seen, sizeof(h_parts), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(landed.data(), gpu_data, landed.size(), hipMemcpyDeviceToHost));
    int wrong = 0;
    for (int k = 0; k < N; k++) wrong += h[k] != 1;
    const bool bytes_ok = std::memcmp(landed.data(), cpu_data, landed.size()) == 0;
    std::printf("  %s: %d of %d entries not marked exactly once, parts %u (want %u), data %s\n", name, wrong, N,
                h_parts, want_parts, bytes_ok ? "ok" : "MISMATCH");
    HIP_OK(hipFree(parts_seen));
    HIP_OK(hipFree(touched));
    HIP_OK(hipFree(gpu_data));
    HIP_OK(hipHostFree(cpu_data));
    return ok && wrong == 0 && h_parts == want_parts && bytes_ok;
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
        gfd::CpuPollingThread* poller = session.get_poller();
        if (!poller) return false;
        print_poller_stats(*poller, session.get_stats().elapsed_ms);
        if (poller->get_descriptors_processed() != (uint64_t)total_tokens ||
            poller->get_total_bytes_copied() != (double)total_size)
            ok = false;
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
    ok = sg_compute_waves<SharedTouch>(sg_shared_kernel, 3, "3 compute waves sharing each list") && ok;
    ok = sg_compute_waves<SoloTouch>(sg_solo_kernel, 1, "3 compute waves, functor without kSharesLists") && ok;
    for (int tiles : {1, 2, 3, 4, 5, 7}) ok = db_tiles(tiles * 64, 64, 16, 128, cus) && ok;
    std::printf("  Verify:    %s\n", ok ? "PASSED" : "FAILED");
    return ok ? 0 : 1;
}
