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
#include <vector>

#include "gfd/hip_shim.h"
#include "gfd/log.h"
#include "sdma.h"

extern "C" const unsigned char gfd_zc_worker_code_object[];
extern "C" const size_t gfd_zc_worker_code_object_size;

namespace gfd {

namespace {

constexpr uint64_t kExitCount = 0xFFFFFF;  // a header count that asks the grid to exit
// The kernel's launch bounds: a prefetch wave and kWavesPerGroup copy waves.
constexpr uint32_t kWorkgroupSize = (ZcWorker::kWavesPerGroup + 1) * 64;
constexpr size_t kKernargBytes = 4096;
constexpr int kMaxGroups = 32;
// words_: the job headers (one cache line each), then from word kProgress
// the workgroups' progress words (one cache line each).
constexpr size_t kProgress = 64;
constexpr size_t kWordsBytes = 4096;
static_assert(ZcWorker::kJobSlots * 8 <= (int)kProgress, "job headers fit before the progress words");
static_assert((kProgress + 8 * kMaxGroups) * 8 <= kWordsBytes, "progress words fit");
static_assert((ZcWorker::kJobSlots & (ZcWorker::kJobSlots - 1)) == 0, "the ring size is a power of two");
// The per-job timeline (64 records of 8 words), then the closing word.
constexpr size_t kTraceWords = 64 * 8;
constexpr size_t kTraceBytes = (kTraceWords + 8) * 8;

// The kernel's explicit arguments, in declaration order at their natural
// alignment.
struct WorkerArgs {
    const uint64_t* headers;
    uint64_t* progress;
    const void* table;
    uint64_t* trace;
    uint32_t num_blocks;
    uint32_t flags;
    uint64_t first_job;
    uint64_t idle_ticks;
    uint64_t epoch;
    uint32_t job_slots;
    uint32_t job_cap;
};
static_assert(sizeof(WorkerArgs) == 72, "gfd_zc_worker arguments");

// One device record: two 16-byte halves, each ending in the job's generation.
struct Record {
    uint64_t dst;
    uint32_t size;
    uint32_t gen;
    uint64_t src;
    uint32_t pad;
    uint32_t gen2;
};
static_assert(sizeof(Record) == 32, "record layout");

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
        // Let posted jobs finish (bounded), then post the exit request.
        wait_until(posted_, 2000000, "the last jobs before exit");
        const uint64_t job = posted_ + 1;
        __atomic_store_n(&words_[(job & (kJobSlots - 1)) * 8], (job << 24) | kExitCount, __ATOMIC_RELEASE);
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
    if (trace_) gfd_hip_free(trace_);
    if (records_) gfd_hip_host_free(records_);
    if (words_) gfd_hip_host_free(words_);
    delete[] list_;
}

int ZcWorker::init(int device, int workgroups, uint32_t idle_ms, int capacity, uint32_t flags) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (ok_) return 0;
    // A job holds at least one and at most kStageRecords records per slot.
    if (workgroups < 1 || workgroups > kMaxGroups || capacity < workgroups * kWavesPerGroup ||
        capacity > workgroups * kWavesPerGroup * kStageRecords)
        return -1;
    workgroups_ = workgroups;
    flags_ = flags;
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
    uint32_t worker_args = 0, worker_priv = 0;
    if (symbol(exe, gpu, "gfd_zc_worker.kd", &worker_object_, &worker_args, &worker_group_, &worker_priv) != 0)
        return -1;
    // The dispatch gives no scratch, and the argument block is fixed.
    if (worker_priv || worker_args < sizeof(WorkerArgs) || worker_args > kKernargBytes) {
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
    if (gfd_hip_host_alloc(&p, kWordsBytes, GFD_HOST_COHERENT) != 0) return -1;
    words_ = static_cast<uint64_t*>(p);
    std::memset(words_, 0, kWordsBytes);
    // Coherent (uncached) for the GPU, as the records change between jobs.
    const size_t rec_bytes = (size_t)kJobSlots * capacity * sizeof(Record);
    if (gfd_hip_host_alloc(&records_, rec_bytes, GFD_HOST_COHERENT) != 0) return -1;
    std::memset(records_, 0, rec_bytes);
    list_ = new SGEntry[capacity];
    capacity_ = capacity;
    // Timeline maxima and the closing word start at 0.
    if (gfd_hip_malloc(&p, kTraceBytes) != 0) return -1;
    trace_ = static_cast<uint64_t*>(p);
    if (gfd_hip_memset_d8((uint64_t)(uintptr_t)trace_, 0, kTraceBytes) != 0 || gfd_hip_device_synchronize() != 0)
        return -1;
    ok_ = true;
    return 0;
}

int ZcWorker::read_timeline(uint64_t* out, int max_jobs) {
    if (!trace_ || !(flags_ & kTrace) || !out || max_jobs <= 0) return 0;
    // Finished jobs' records do not change while the grid waits for the next.
    std::lock_guard<std::recursive_mutex> lock(mu_);
    const int n = max_jobs < 64 ? max_jobs : 64;
    std::vector<uint64_t> all(kTraceWords);
    if (gfd_hip_memcpy_d2h(all.data(), (uint64_t)(uintptr_t)trace_, all.size() * 8) != 0) return 0;
    // Newest first: the last job, then the ones before it.
    int k = 0;
    for (int i = 0; i < n && (uint64_t)i < posted_; i++) {
        const uint64_t job = posted_ - (uint64_t)i;
        const uint64_t* r = &all[(job & 63u) * 8];
        if (r[6] != job) break;
        std::memcpy(out + (size_t)k * 8, r, 8 * sizeof(uint64_t));
        k++;
    }
    return k;
}

bool ZcWorker::grid_finished() const { return hsa_signal_load_scacquire(as_signal(signal_)) == 0; }

int ZcWorker::launch() {
    hsa_queue_t* q = static_cast<hsa_queue_t*>(queue_);
    auto* wa = static_cast<WorkerArgs*>(kernarg_);
    // The grid starts at the first job not done.  A new epoch per dispatch:
    // a closing word left by an earlier grid never matches it.
    *wa = WorkerArgs{words_,         &words_[kProgress], records_,          trace_,  (uint32_t)workgroups_, flags_,
                     completed_ + 1, idle_ticks_,        launches_ + 1,     kJobSlots, (uint32_t)capacity_};
    hsa_signal_store_relaxed(as_signal(signal_), 1);
    if (dispatch(q, worker_object_, worker_group_, wa, kWorkgroupSize, kWorkgroupSize * (uint32_t)workgroups_,
                 as_signal(signal_)) != 0) {
        GFD_LOG_ERROR("zero-copy worker: dispatch failed\n");
        return -1;
    }
    dispatched_ = true;
    launches_++;
    return 0;
}

bool ZcWorker::poll() {
    const uint64_t* progress = &words_[kProgress];
    for (int pass = 0; pass < 2; pass++) {
        // A progress word counts the jobs its workgroup finished in order; a
        // grid dispatched again may store smaller numbers for jobs it runs a
        // second time, so completed_ never goes back.
        uint64_t m = ~0ull;
        for (int b = 0; b < workgroups_; b++) {
            const uint64_t v = __atomic_load_n(&progress[b * 8], __ATOMIC_ACQUIRE);
            m = v < m ? v : m;
        }
        if (m > completed_) completed_ = m > posted_ ? posted_ : m;
        if (completed_ >= posted_ || !dispatched_ || !grid_finished()) return true;
        // The grid has ended (idle) with jobs left; read the words once more,
        // as it may have finished them just before it ended.
        if (pass == 1) return launch() == 0;
    }
    return true;
}

bool ZcWorker::done(uint64_t job) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (completed_ >= job) return true;
    if (!ok_) return false;
    poll();
    return completed_ >= job;
}

int ZcWorker::wait_until(uint64_t job, uint64_t timeout_us, const char* what) {
    const auto t0 = std::chrono::steady_clock::now();
    for (unsigned i = 1;; i++) {
        if (completed_ >= job) return 0;
        if (!poll()) {
            ok_ = false;
            return -1;
        }
        if (completed_ >= job) return 0;
        _mm_pause();
        if ((i & 1023) == 0 &&
            (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0)
                    .count() > timeout_us) {
            GFD_LOG_ERROR("zero-copy worker: %s not done in %llu us; the worker is off\n", what,
                          (unsigned long long)timeout_us);
            ok_ = false;
            return -1;
        }
    }
}

int ZcWorker::wait(uint64_t job, uint64_t timeout_us) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (completed_ >= job) return 0;
    if (!ok_) return -1;
    return wait_until(job, timeout_us, "a job");
}

uint64_t ZcWorker::post(int count, uint64_t timeout_us, const SGEntry* list) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (!ok_ || count <= 0 || count > capacity_) return 0;
    const SGEntry* in = list ? list : list_;
    for (int i = 0; i < count; i++)
        if (in[i].size > 0xFFFFFFFFull) return 0;
    const uint64_t job = posted_ + 1;
    // The job's ring slot held job - kJobSlots, which every workgroup must
    // have finished (and so stopped reading).
    if (job > (uint64_t)kJobSlots && wait_until(job - kJobSlots, timeout_us, "a free job slot") != 0) return 0;
    if ((!dispatched_ || grid_finished()) && launch() != 0) {
        ok_ = false;
        return 0;
    }
    // A job of at most one record per slot stores record s (slot s: wave
    // s / workgroups of workgroup s % workgroups) at region position
    // (s % workgroups) * 8 + s / workgroups, so each workgroup reads its
    // records as one contiguous run; a larger job is stored in order.  Each
    // half's generation is stored after its other fields (release stores, in
    // order on x86), so a half read with this generation in one request holds
    // this job's fields.
    const bool by_slot = count <= waves();
    const uint32_t gen = (uint32_t)(job & 0xFFFFFFu);
    auto* region = static_cast<Record*>(records_) + (size_t)(job & (kJobSlots - 1)) * capacity_;
    for (int i = 0; i < count; i++) {
        Record& r = region[by_slot ? (i % workgroups_) * kWavesPerGroup + i / workgroups_ : i];
        r.dst = (uint64_t)in[i].dst;
        r.size = (uint32_t)in[i].size;
        r.src = (uint64_t)(uintptr_t)in[i].src;
        r.pad = 0;
        __atomic_store_n(&r.gen, gen, __ATOMIC_RELEASE);
        __atomic_store_n(&r.gen2, gen, __ATOMIC_RELEASE);
    }
    __atomic_store_n(&words_[(job & (kJobSlots - 1)) * 8], (job << 24) | (uint64_t)count, __ATOMIC_RELEASE);
    posted_ = job;
    return job;
}

int ZcWorker::run(int count, uint64_t timeout_us) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (count == 0) return ok_ ? 0 : -1;
    const uint64_t job = post(count, timeout_us);
    return job ? wait(job, timeout_us) : -1;
}

}  // namespace gfd
