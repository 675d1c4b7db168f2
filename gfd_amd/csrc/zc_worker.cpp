// ZcWorker (see zc_worker.h): the host side of the persistent zero-copy
// worker.  The device code (aql/zc_worker.hip) is built into a raw gfx950
// code object that the build embeds as gfd_zc_worker_code_object; it is
// loaded here through the HSA runtime and dispatched with AQL packets on a
// queue of this object's own.
#include "zc_worker.h"

#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <immintrin.h>

#include <chrono>
#include <cstring>

#include "gfd/hip_shim.h"
#include "gfd/log.h"
#include "sdma.h"

extern "C" const unsigned char gfd_zc_worker_code_object[];
extern "C" const size_t gfd_zc_worker_code_object_size;

namespace gfd {

namespace {

constexpr uint64_t kExitJob = ~0ull;
constexpr uint32_t kWorkgroupSize = 256;  // 4 waves, as the kernel's launch bounds
constexpr size_t kKernargBytes = 4096;
constexpr size_t kResetArgs = 0, kWorkerArgs = 1024;  // offsets in the kernarg block
constexpr size_t kStateBytes = 256;

// Explicit arguments of the two kernels, in declaration order at their
// natural alignment.
struct WorkerArgs {
    const uint64_t* doorbell;
    uint64_t* done;
    const void* table;
    void* state;
    uint32_t num_blocks;
    uint32_t pad;
    uint64_t last_job;
    uint64_t idle_ticks;
};
static_assert(sizeof(WorkerArgs) == 56, "gfd_zc_worker arguments");
struct ResetArgs {
    void* state;
    uint64_t last_job;
};

hsa_status_t find_kernarg_pool(hsa_amd_memory_pool_t p, void* data) {
    hsa_amd_segment_t seg;
    if (hsa_amd_memory_pool_get_info(p, HSA_AMD_MEMORY_POOL_INFO_SEGMENT, &seg) != HSA_STATUS_SUCCESS ||
        seg != HSA_AMD_SEGMENT_GLOBAL)
        return HSA_STATUS_SUCCESS;
    uint32_t flags = 0;
    hsa_amd_memory_pool_get_info(p, HSA_AMD_MEMORY_POOL_INFO_GLOBAL_FLAGS, &flags);
    auto* out = static_cast<hsa_amd_memory_pool_t*>(data);
    if ((flags & HSA_AMD_MEMORY_POOL_GLOBAL_FLAG_KERNARG_INIT) && !out->handle) *out = p;
    return HSA_STATUS_SUCCESS;
}

hsa_signal_t as_signal(uint64_t h) {
    hsa_signal_t s;
    s.handle = h;
    return s;
}

int symbol(hsa_executable_t exe, hsa_agent_t gpu, const char* name, uint64_t* object, uint32_t* kernarg,
           uint32_t* group, uint32_t* priv) {
    hsa_executable_symbol_t sym;
    if (hsa_executable_get_symbol_by_name(exe, name, &gpu, &sym) != HSA_STATUS_SUCCESS) return -1;
    if (hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, object) != HSA_STATUS_SUCCESS ||
        hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE, kernarg) !=
            HSA_STATUS_SUCCESS ||
        hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE, group) !=
            HSA_STATUS_SUCCESS ||
        hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE, priv) !=
            HSA_STATUS_SUCCESS)
        return -1;
    return 0;
}

// One AQL kernel dispatch packet: 1-D grid of `grid` work-items in workgroups
// of `wg`, ordered after every earlier packet of the queue (barrier bit),
// with system-scope acquire and release fences.
int dispatch(hsa_queue_t* q, uint64_t object, uint32_t group, void* kernarg, uint32_t wg, uint32_t grid,
             hsa_signal_t completion) {
    const uint64_t idx = hsa_queue_add_write_index_relaxed(q, 1);
    // At most two packets are ever in flight on this queue of >= 64 slots.
    for (uint64_t n = 0; idx - hsa_queue_load_read_index_scacquire(q) >= q->size; n++)
        if (n > (1ull << 30)) return -1;
    auto* p = static_cast<hsa_kernel_dispatch_packet_t*>(q->base_address) + (idx & (q->size - 1));
    std::memset(reinterpret_cast<char*>(p) + 4, 0, sizeof(*p) - 4);
    p->workgroup_size_x = (uint16_t)wg;
    p->workgroup_size_y = 1;
    p->workgroup_size_z = 1;
    p->grid_size_x = grid;
    p->grid_size_y = 1;
    p->grid_size_z = 1;
    p->private_segment_size = 0;
    p->group_segment_size = group;
    p->kernel_object = object;
    p->kernarg_address = kernarg;
    p->completion_signal = completion;
    const uint32_t header = (HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) |
                            (1u << HSA_PACKET_HEADER_BARRIER) |
                            (HSA_FENCE_SCOPE_SYSTEM << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
                            (HSA_FENCE_SCOPE_SYSTEM << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE);
    const uint32_t setup = 1u << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS;
    __atomic_store_n(reinterpret_cast<uint32_t*>(p), header | (setup << 16), __ATOMIC_RELEASE);
    hsa_signal_store_screlease(q->doorbell_signal, (hsa_signal_value_t)idx);
    return 0;
}

}  // namespace

ZcWorker::ZcWorker() = default;

ZcWorker::~ZcWorker() {
    hsa_queue_t* q = static_cast<hsa_queue_t*>(queue_);
    if (dispatched_ && signal_ && !grid_finished()) {
        __atomic_store_n(&words_[0], kExitJob, __ATOMIC_RELEASE);
        if (hsa_signal_wait_scacquire(as_signal(signal_), HSA_SIGNAL_CONDITION_LT, 1, 5000000000ull,
                                      HSA_WAIT_STATE_ACTIVE) != 0) {
            // Still running: leave every resource it uses in place.
            GFD_LOG_ERROR("zero-copy worker did not exit; its resources are kept\n");
            return;
        }
    }
    if (q) hsa_queue_destroy(q);
    if (signal_) hsa_signal_destroy(as_signal(signal_));
    if (executable_) hsa_executable_destroy(hsa_executable_t{executable_});
    if (reader_) hsa_code_object_reader_destroy(hsa_code_object_reader_t{reader_});
    if (kernarg_) hsa_amd_memory_pool_free(kernarg_);
    if (state_) gfd_hip_free(state_);
    if (table_) gfd_hip_host_free(table_);
    if (words_) gfd_hip_host_free(words_);
}

int ZcWorker::init(int device, int workgroups, uint32_t idle_ms, int capacity) {
    if (ok_) return 0;
    if (workgroups < 1 || capacity < 1 || capacity >= (1 << 24)) return -1;
    workgroups_ = workgroups;
    idle_ticks_ = (uint64_t)(idle_ms ? idle_ms : 1) * 100000ull;  // 100 MHz wall clock
    if (find_hsa_agents(device, &gpu_agent_, &cpu_agent_) != 0) return -1;
    hsa_agent_t gpu{gpu_agent_}, cpu{cpu_agent_};
    hsa_code_object_reader_t reader;
    if (hsa_code_object_reader_create_from_memory(gfd_zc_worker_code_object, gfd_zc_worker_code_object_size,
                                                  &reader) != HSA_STATUS_SUCCESS)
        return -1;
    reader_ = reader.handle;
    hsa_executable_t exe;
    if (hsa_executable_create_alt(HSA_PROFILE_FULL, HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT, nullptr, &exe) !=
        HSA_STATUS_SUCCESS)
        return -1;
    executable_ = exe.handle;
    if (hsa_executable_load_agent_code_object(exe, gpu, reader, nullptr, nullptr) != HSA_STATUS_SUCCESS ||
        hsa_executable_freeze(exe, nullptr) != HSA_STATUS_SUCCESS)
        return -1;
    uint32_t reset_args = 0, worker_args = 0, reset_priv = 0, worker_priv = 0;
    if (symbol(exe, gpu, "gfd_zc_worker_reset.kd", &reset_object_, &reset_args, &reset_group_, &reset_priv) != 0 ||
        symbol(exe, gpu, "gfd_zc_worker.kd", &worker_object_, &worker_args, &worker_group_, &worker_priv) != 0)
        return -1;
    // The dispatches give no scratch, and the argument blocks are fixed.
    if (reset_priv || worker_priv || reset_args < sizeof(ResetArgs) || reset_args > kWorkerArgs - kResetArgs ||
        worker_args < sizeof(WorkerArgs) || worker_args > kKernargBytes - kWorkerArgs) {
        GFD_LOG_ERROR("zero-copy worker: unexpected kernel segment sizes\n");
        return -1;
    }
    hsa_amd_memory_pool_t pool{0};
    hsa_amd_agent_iterate_memory_pools(cpu, find_kernarg_pool, &pool);
    if (!pool.handle || hsa_amd_memory_pool_allocate(pool, kKernargBytes, 0, &kernarg_) != HSA_STATUS_SUCCESS ||
        hsa_amd_agents_allow_access(1, &gpu, nullptr, kernarg_) != HSA_STATUS_SUCCESS)
        return -1;
    std::memset(kernarg_, 0, kKernargBytes);
    hsa_queue_t* q = nullptr;
    if (hsa_queue_create(gpu, 64, HSA_QUEUE_TYPE_SINGLE, nullptr, nullptr, UINT32_MAX, UINT32_MAX, &q) !=
        HSA_STATUS_SUCCESS)
        return -1;
    queue_ = q;
    // Polled by this object, never waited on through an interrupt event.
    hsa_signal_t s;
    if (hsa_amd_signal_create(0, 0, nullptr, HSA_AMD_SIGNAL_AMD_GPU_ONLY, &s) != HSA_STATUS_SUCCESS) return -1;
    signal_ = s.handle;
    void* p = nullptr;
    if (gfd_hip_host_alloc(&p, 4096, GFD_HOST_COHERENT) != 0) return -1;
    words_ = static_cast<uint64_t*>(p);
    std::memset(words_, 0, 4096);
    // Coherent (uncached) for the GPU, as the records change between jobs.
    if (gfd_hip_host_alloc(&p, (size_t)capacity * sizeof(SGEntry), GFD_HOST_COHERENT) != 0) return -1;
    table_ = static_cast<SGEntry*>(p);
    capacity_ = capacity;
    if (gfd_hip_malloc(&state_, kStateBytes) != 0) return -1;
    ok_ = true;
    return 0;
}

bool ZcWorker::grid_finished() const { return hsa_signal_load_scacquire(as_signal(signal_)) == 0; }

int ZcWorker::launch() {
    hsa_queue_t* q = static_cast<hsa_queue_t*>(queue_);
    auto* ra = reinterpret_cast<ResetArgs*>(static_cast<char*>(kernarg_) + kResetArgs);
    ra->state = state_;
    ra->last_job = last_done_;
    auto* wa = reinterpret_cast<WorkerArgs*>(static_cast<char*>(kernarg_) + kWorkerArgs);
    *wa = WorkerArgs{&words_[0], &words_[8], table_, state_, (uint32_t)workgroups_, 0, last_done_, idle_ticks_};
    hsa_signal_store_relaxed(as_signal(signal_), 1);
    if (dispatch(q, reset_object_, reset_group_, ra, 64, 64, hsa_signal_t{0}) != 0 ||
        dispatch(q, worker_object_, worker_group_, wa, kWorkgroupSize, kWorkgroupSize * (uint32_t)workgroups_,
                 as_signal(signal_)) != 0) {
        GFD_LOG_ERROR("zero-copy worker: dispatch failed\n");
        return -1;
    }
    dispatched_ = true;
    launches_++;
    return 0;
}

int ZcWorker::run(int count, uint64_t timeout_us) {
    if (!ok_ || count < 0 || count > capacity_) return -1;
    if (count == 0) return 0;
    if ((!dispatched_ || grid_finished()) && launch() != 0) return -1;
    gen_ = (gen_ + 1) & 0xFFFFu;
    if (gen_ == 0) gen_ = 1;
    const uint64_t job = (uint64_t)gen_ | ((uint64_t)count << 16);
    // The records are in place (this thread's earlier stores); the release
    // keeps them ahead of the doorbell.
    __atomic_store_n(&words_[0], job, __ATOMIC_RELEASE);
    jobs_++;
    const auto t0 = std::chrono::steady_clock::now();
    for (unsigned i = 1;; i++) {
        if (__atomic_load_n(&words_[8], __ATOMIC_ACQUIRE) == job) {
            last_done_ = job;
            return 0;
        }
        _mm_pause();
        if ((i & 1023) != 0) continue;
        // The grid may have ended (idle) just before the doorbell: start it again.
        if (grid_finished()) {
            if (__atomic_load_n(&words_[8], __ATOMIC_ACQUIRE) == job) continue;
            if (launch() != 0) return -1;
        }
        if ((uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0)
                .count() > timeout_us) {
            GFD_LOG_ERROR("zero-copy worker: job of %d records not done in %llu us\n", count,
                          (unsigned long long)timeout_us);
            return -1;
        }
    }
}

}  // namespace gfd
