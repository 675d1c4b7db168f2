// CpuPollingThread: lifecycle, resources and the descriptor-ring poller
// (declaration: include/gfd/cpu_polling.h).
//
// Reference behaviour kept (src/cpu_polling.cpp:37-490,
// src/batch_processor.cpp:307-723):
//   * a descriptor is consumed when sequence == read_idx + 1 (acquire); the
//     poller zeroes sequence (release) and advances read_idx;
//   * batches close at BATCH_THRESHOLD entries (BATCH_THRESHOLD_SMALL when the
//     first entry is <= 2 KB), at MAX_BATCH_SIZE, on LAST_IN_BATCH / URGENT /
//     LAST_IN_TILE (tiled and SG modes), or after a 4096-pause gap with no
//     new descriptor;
//   * a dst-contiguous, src-scattered batch is gathered into the next of
//     NUM_STAGING_BUFS rotating pinned buffers and copied as one range;
//   * done_idx only moves forward, and only past slots whose copies finished;
//   * tiled mode: per-tile cumulative progress; SG mode: one list at a time,
//     d_list_done[list_id] = 1 after the list's copies.
// MI355X design differences:
//   * copies are SDMA transfers tracked by fences (no GPU stream is involved,
//     so a kernel spinning on done_idx can never block them);
//   * done_idx advances per batch as soon as that batch's copies finish;
//   * batch gathers are pipelined: each staging chunk is copied as soon as the
//     worker pool has filled it;
//   * HBM flags are 8-byte SDMA writes chained behind the data copies on the
//     engine; flags in host memory are written by this thread on completion.
#include "gfd/cpu_polling.h"

#include <immintrin.h>
#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <vector>

#include "dst_runs.h"
#include "gather_engine.h"
#include "gfd/pcie_topology.h"
#include "gfd/sg_task_queue.h"
#include "gfd/staging_pool.h"
#include "zc_worker.h"

namespace gfd {

// Ring of completion points, oldest at `tail`.
struct CpuPollingThread::CompletionFifo {
    static constexpr int N = 64;
    CompletionSlot slots[N];
    int head = 0;
    int tail = 0;
    int count = 0;
};

namespace {

inline void cpu_relax() { _mm_pause(); }

inline uint64_t now_us() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

size_t env_size(const char* name, size_t dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    char* end = nullptr;
    unsigned long long x = std::strtoull(v, &end, 0);
    return (end && end != v) ? (size_t)x : dflt;
}

void pin_self(int cpu) {
    if (cpu < 0) return;
    cpu_set_t cs;
    CPU_ZERO(&cs);
    CPU_SET(cpu, &cs);
    pthread_setaffinity_np(pthread_self(), sizeof(cs), &cs);
}

struct ChunkCtx {
    CpuPollingThread* self;
    CopyEngineManager* ce;
    DevicePtr dst0;
    const char* staging;
    int channels;
    int err;
};

void issue_chunk(void* p, int chunk, size_t off, size_t len) {
    ChunkCtx* c = (ChunkCtx*)p;
    int e = c->ce->submit_on_channel(chunk % c->channels, c->dst0 + off, c->staging + off, len);
    if (e && !c->err) c->err = e;
    c->self->trace(CpuPollingThread::TRACE_CHUNK, (uint32_t)chunk, len);
}

}  // namespace

CpuPollingThread::CpuPollingThread(DescriptorQueue* queue, void* gpu_base, void* cpu_base,
                                   size_t total_cpu_size, bool use_ce, int numa_node,
                                   int core_offset, int num_ce_channels, int exclusive_core_base,
                                   int exclusive_core_count)
    : queue_(queue),
      gpu_base_(gpu_base),
      cpu_base_(cpu_base),
      total_cpu_size_(total_cpu_size),
      use_ce_(use_ce),
      numa_node_(numa_node),
      core_offset_(core_offset),
      num_ce_channels_(num_ce_channels),
      exclusive_core_base_(exclusive_core_base),
      exclusive_core_count_(exclusive_core_count) {
    gfd_hip_get_device(&device_);
    direct_chunk_bytes_ = env_size("GFD_DIRECT_CHUNK_BYTES", direct_chunk_bytes_);
    direct_zc_max_bytes_ = env_size("GFD_DIRECT_ZC_MAX_BYTES", direct_zc_max_bytes_);
    direct_zc_min_bytes_ = env_size("GFD_DIRECT_ZC_MIN_BYTES", direct_zc_min_bytes_);
    direct_zc_head_bytes_ = env_size("GFD_DIRECT_ZC_HEAD_BYTES", direct_zc_head_bytes_);
    worker_wanted_ = env_size("GFD_ZC_WORKER", 0) != 0;
    worker_queue_max_bytes_ = env_size("GFD_ZC_WORKER_QUEUE_MAX_BYTES", worker_queue_max_bytes_);
    fifo_ = new CompletionFifo();
    if (env_size("GFD_TRACE", 0)) set_trace(true);
}

CpuPollingThread::~CpuPollingThread() {
    stop_hook_ = nullptr;  // its owner may be half destroyed
    stop();
    delete worker_;  // ends its grid
    worker_ = nullptr;
    delete gather_;
    gather_ = nullptr;
    gfd_hip_set_device(device_);
    ce_manager_.wait_completion();
    direct_ce_manager_.wait_completion();
    delete fifo_;
    fifo_ = nullptr;
    if (staging_pool_set_ >= 0) {
        StagingPool::instance().release_buffers(staging_pool_set_);
        staging_pool_set_ = -1;
    } else if (staging_owned_) {
        for (int b = 0; b < NUM_STAGING_BUFS; b++) StagingPool::free_pinned(staging_bufs_[b]);
    }
    for (int b = 0; b < NUM_STAGING_BUFS; b++) staging_bufs_[b] = nullptr;
    StagingPool::free_pinned(direct_staging_);
    direct_staging_ = nullptr;
    if (signal_values_) gfd_hip_host_free(signal_values_);
    signal_values_ = nullptr;
    if (zc_stream_) {
        gfd_hip_stream_synchronize(zc_stream_);
        gfd_hip_stream_destroy(zc_stream_);
        zc_stream_ = nullptr;
    }
    if (zc_table_) gfd_hip_host_free(zc_table_);
    zc_table_ = nullptr;
    if (zc_src_table_) gfd_hip_host_free(zc_src_table_);
    zc_src_table_ = nullptr;
    if (zc_done_) gfd_hip_host_free(zc_done_);
    zc_done_ = nullptr;
    if (zc_counter_) gfd_hip_free(zc_counter_);
    zc_counter_ = nullptr;
    ce_manager_.shutdown();
    direct_ce_manager_.shutdown();
}

int CpuPollingThread::num_gather_workers() const { return gather_ ? gather_->num_workers() : 0; }

// The worker's grid: by default 8 workgroups of 8 copy waves (64 waves, the
// zero-copy kernels' short-list width), one workgroup per XCD; up to 64
// records per copy wave in a job (4096: a Queue batch holds at most
// BATCH_THRESHOLD entries).  GFD_ZC_WORKER_GROUPS sets the workgroups
// (1-32), GFD_ZC_WORKER_TRACE=1 records the device timeline.
bool CpuPollingThread::ensure_worker() {
    if (worker_) return true;
    auto* w = new ZcWorker();
    const uint32_t idle_ms = (uint32_t)env_size("GFD_ZC_WORKER_IDLE_MS", 100);
    const int groups = (int)std::min<size_t>(std::max<size_t>(env_size("GFD_ZC_WORKER_GROUPS", 8), 1), 32);
    const uint32_t flags = env_size("GFD_ZC_WORKER_TRACE", 0) ? ZcWorker::kTrace : 0u;
    const int capacity = groups * ZcWorker::kWavesPerGroup * ZcWorker::kStageRecords;
    if (gfd_hip_set_device(device_) != 0 || w->init(device_, groups, idle_ms, capacity, flags) != 0) {
        GFD_LOG_ERROR("zero-copy worker set-up failed; it stays off\n");
        delete w;
        return false;
    }
    worker_ = w;
    worker_posted_ = worker_done_seen_ = 0;
    return true;
}

int CpuPollingThread::set_zero_copy_worker(bool on) {
    if (running_.load(std::memory_order_acquire)) {
        GFD_LOG_ERROR("set_zero_copy_worker: stop the polling thread first\n");
        return -1;
    }
    std::lock_guard<std::mutex> direct_lock(direct_mutex_);
    if (!on) {
        delete worker_;
        worker_ = nullptr;
        worker_wanted_ = false;
        worker_posted_ = worker_done_seen_ = 0;
        return 0;
    }
    worker_wanted_ = true;
    return ensure_worker() ? 0 : -1;
}

uint64_t CpuPollingThread::zero_copy_worker_jobs() const { return worker_ ? worker_->jobs() : 0; }
uint64_t CpuPollingThread::zero_copy_worker_launches() const { return worker_ ? worker_->launches() : 0; }
int CpuPollingThread::zero_copy_worker_timeline(uint64_t* out, int max_jobs) {
    return worker_ ? worker_->read_timeline(out, max_jobs) : 0;
}

// Queue path: a batch whose sources are pinned and whose destinations lie in
// device memory goes to the worker as one job.  In plain Queue mode the job
// is only posted: the batch's completion slot waits for it before done_idx
// passes the batch.  Tiled and SG modes write their flags with copy-engine
// packets ordered after the engines' copies only, so there the job is waited
// for here.  False if the batch does not qualify or the worker failed; the
// caller then stages it for the copy engines.
bool CpuPollingThread::queue_worker_copy(const SGEntry* e, int count, size_t total) {
    if (!worker_ || !worker_->ok() || total > worker_queue_max_bytes_ || count > worker_->capacity()) return false;
    uintptr_t lo = 1, hi = 0;
    for (int i = 0; i < count; i++) {
        if (e[i].size == 0) continue;
        const uintptr_t a = (uintptr_t)e[i].src, b = a + e[i].size;
        if (a < lo || b > hi) {
            if (!ce_manager_.host_source_ok(e[i].src, e[i].size)) return false;
            ce_manager_.last_pinned_range(&lo, &hi);
            if (a < lo || b > hi) lo = a, hi = b;
        }
        const uint64_t d = e[i].dst, de = d + e[i].size;
        if (d < queue_dst_lo_ || de > queue_dst_hi_) {
            uint64_t base = 0, size = 0;
            if (!gfd_hip_device_range(d, &base, &size) || de > base + size) return false;
            queue_dst_lo_ = base;
            queue_dst_hi_ = base + size;
        }
    }
    trace(TRACE_ZC_CHECKED, (uint32_t)count, total);
    static const uint64_t timeout_us = (uint64_t)env_size("GFD_DIRECT_TIMEOUT_MS", 10000) * 1000ull;
    std::lock_guard<std::recursive_mutex> lock(worker_->mutex());
    uint64_t job = 0;
    if (count >= worker_->waves()) {
        // At least one entry per slot: nothing to cut, posted as it is.
        trace(TRACE_ZC_LAUNCH, (uint32_t)count, total);
        job = worker_->post(count, timeout_us, e);
    } else {
        bool cut = false;
        const int n =
            zc_fill_sg_table(e, count, total, worker_->table(), worker_->capacity(), &cut, worker_->waves());
        trace(TRACE_ZC_LAUNCH, (uint32_t)count, total);
        job = worker_->post(n, timeout_us);
    }
    if (job != 0 && (tiled_queue_ || sg_queue_)) {
        if (worker_->wait(job, timeout_us) != 0) GFD_LOG_ERROR("zero-copy worker: queue batch failed\n");
        trace(TRACE_ZC_DONE, 0, job);
    }
    if (job == 0) {
        GFD_LOG_ERROR("zero-copy worker: queue batch not posted; staging it\n");
        return false;
    }
    worker_posted_ = job;
    return true;
}

void CpuPollingThread::set_trace(bool on) {
    std::lock_guard<std::mutex> lock(trace_mutex_);
    if (on && trace_buf_.empty()) trace_buf_.resize(TRACE_CAP);
    trace_on_.store(on, std::memory_order_release);
}

void CpuPollingThread::set_copy_timing(bool on) {
    if (ce_manager_.is_initialized()) ce_manager_.set_copy_timing(on);
    if (direct_ce_manager_.is_initialized()) direct_ce_manager_.set_copy_timing(on);
}

int CpuPollingThread::read_copy_times(CopyTiming* out, int max) {
    int n = 0;
    CopyEngineManager* mgrs[2] = {&ce_manager_, &direct_ce_manager_};
    for (uint32_t path = 0; path < 2 && n < max; path++) {
        if (!mgrs[path]->is_initialized()) continue;
        CopyEngineManager::CopyTime buf[256];
        for (;;) {
            const size_t want = std::min<size_t>(256, (size_t)(max - n));
            if (want == 0) break;
            const size_t got = mgrs[path]->read_copy_times(buf, want);
            for (size_t i = 0; i < got; i++)
                out[n++] = CopyTiming{buf[i].seq, buf[i].bytes, buf[i].start_ns, buf[i].end_ns,
                                      buf[i].channel, buf[i].engine, path, 0};
            if (got < want) break;
        }
    }
    return n;
}

uint64_t CpuPollingThread::copy_clock_ns() const {
    if (direct_ce_manager_.is_initialized()) return direct_ce_manager_.copy_clock_ns();
    return ce_manager_.copy_clock_ns();
}

void CpuPollingThread::trace(uint32_t kind, uint32_t a, uint64_t b) {
    if (!trace_on_.load(std::memory_order_relaxed)) return;
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    trace_at((uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec, kind, a, b);
}

void CpuPollingThread::trace_at(uint64_t t_ns, uint32_t kind, uint32_t a, uint64_t b) {
    if (!trace_on_.load(std::memory_order_relaxed)) return;
    std::lock_guard<std::mutex> lock(trace_mutex_);
    if (trace_buf_.empty()) return;
    if (trace_head_ - trace_tail_ == (uint64_t)TRACE_CAP) trace_tail_++;  // overwrite the oldest
    trace_buf_[trace_head_ % TRACE_CAP] = TraceEvent{t_ns, kind, a, b};
    trace_head_++;
}

int CpuPollingThread::read_trace(TraceEvent* out, int max) {
    std::lock_guard<std::mutex> lock(trace_mutex_);
    int n = 0;
    while (n < max && trace_tail_ < trace_head_) out[n++] = trace_buf_[trace_tail_++ % TRACE_CAP];
    return n;
}

void CpuPollingThread::set_gather_slice_bytes(size_t b) {
    slice_bytes_ = b;
    if (gather_) gather_->set_slice_bytes(b);
}

bool CpuPollingThread::choose_cpus() {
    if (cpus_chosen_) return true;
    GpuTopology topo = discover_gpu_topology(device_);
    if (numa_node_ < 0) numa_node_ = topo.numa_node;
    // Default worker count: with an explicit core range, the reference rule
    // (up to 15); otherwise half of the CPUs this process may use, so the
    // application thread, the GPU runtime's threads and the poller keep cores
    // of their own (a handful of AVX-512 streams already outrun the link).
    int dflt = MAX_GATHER_WORKERS;
    if (!(exclusive_core_base_ >= 0 && exclusive_core_count_ > 0)) {
        const int avail = (int)allowed_cpus().size();
        dflt = std::max(1, std::min(MAX_GATHER_WORKERS, avail / 2));
    }
    int cap = (int)env_size("GFD_NUM_GATHER_WORKERS", (size_t)dflt);
    if (cap > MAX_GATHER_WORKERS) cap = MAX_GATHER_WORKERS;
    std::vector<int> cpus = pick_cpus(topo, 1 + cap, exclusive_core_base_, exclusive_core_count_);
    if (cpus.empty()) cpus.push_back(-1);
    poller_cpu_ = cpus[0];
    worker_cpus_.assign(cpus.begin() + 1, cpus.end());
    cpus_chosen_ = true;
    return true;
}

bool CpuPollingThread::start_workers() {
    if (gather_) return true;
    choose_cpus();
    gather_ = new GatherEngine(worker_cpus_);
    if (!slice_bytes_) slice_bytes_ = env_size("GFD_GATHER_SLICE_BYTES", 128 * 1024);
    gather_->set_slice_bytes(slice_bytes_);
    gather_->set_first_chunk_bytes(env_size("GFD_FIRST_CHUNK_BYTES", 0));
    gather_->set_chunk_ramp(env_size("GFD_CHUNK_RAMP", 1) != 0);
    GFD_LOG_INFO("gather workers: %d (poller CPU %d, NUMA %d)\n", gather_->num_workers(), poller_cpu_,
                 numa_node_);
    return true;
}

bool CpuPollingThread::init_copy_engine() {
    if (!use_ce_) {
        GFD_LOG_ERROR("use_ce=false is not supported: copies always use the SDMA engines\n");
        return false;
    }
    if (gfd_hip_set_device(device_) != 0) return false;
    choose_cpus();
    if (ce_manager_.init(device_, num_ce_channels_) != 0) {
        GFD_LOG_ERROR("copy engine init failed\n");
        return false;
    }
    if (!signal_values_) {
        if (gfd_hip_host_alloc((void**)&signal_values_, sizeof(uint64_t) * SIGNAL_SLOTS, GFD_HOST_DEFAULT) != 0) {
            GFD_LOG_ERROR("signal value buffer allocation failed\n");
            return false;
        }
        std::memset(signal_values_, 0, sizeof(uint64_t) * SIGNAL_SLOTS);
    }

    staging_buffer_size_ = total_cpu_size_;
    int got = 0;
    auto& pool = StagingPool::instance();
    if (pool.is_initialized() && staging_buffer_size_ <= pool.buffer_size()) {
        int set = pool.acquire_buffers(staging_buffer_size_, numa_node_);
        if (set >= 0) {
            char* bufs[StagingPool::BUFS_PER_SET];
            size_t sz = 0;
            bool hp = false;
            pool.get_buffers(set, bufs, sz, hp);
            staging_pool_set_ = set;
            for (int b = 0; b < NUM_STAGING_BUFS && b < StagingPool::BUFS_PER_SET; b++) staging_bufs_[b] = bufs[b];
            got = NUM_STAGING_BUFS;
        }
    }
    if (got == 0 && staging_buffer_size_ > 0) {
        for (int b = 0; b < NUM_STAGING_BUFS; b++) {
            staging_bufs_[b] = StagingPool::alloc_pinned(staging_buffer_size_, numa_node_, nullptr);
            if (!staging_bufs_[b]) break;
            got++;
        }
        staging_owned_ = true;
    }
    num_staging_bufs_ = got;
    for (int b = 0; b < NUM_STAGING_BUFS; b++) staging_fence_[b] = 0;
    for (int b = 0; b < got; b++) ce_manager_.trust_range(staging_bufs_[b], staging_buffer_size_);
    if (worker_wanted_) ensure_worker();
    GFD_LOG_INFO("queue staging: %d x %zu bytes (NUMA %d), %d copy channel(s), SDMA engines 0x%x\n", got,
                 staging_buffer_size_, numa_node_, ce_manager_.num_channels(), ce_manager_.sdma_engine_mask());
    return start_workers();
}

void CpuPollingThread::start() {
    if (running_.load(std::memory_order_acquire)) return;
    if (!queue_) {
        GFD_LOG_ERROR("start(): no descriptor queue\n");
        return;
    }
    if (!ce_manager_.is_initialized()) {
        GFD_LOG_ERROR("start(): init_copy_engine() has not succeeded\n");
        return;
    }
#ifndef GFD_HOST_EMULATION
    // Switched off: with an SG task queue set, the process aborted on MI355X
    // ("stack smashing detected" on a non-Python thread) in both runs made,
    // one with lists posted by a kernel and one by a CPU producer, and the
    // cause has not been found.  The host emulation build keeps the mode so
    // that its logic stays tested.
    if (sg_queue_) {
        GFD_LOG_ERROR("start(): SG task-queue mode is switched off in this library\n");
        return;
    }
#endif
    running_.store(true, std::memory_order_release);
    thread_ = std::thread(&CpuPollingThread::polling_loop, this);
}

void CpuPollingThread::stop() {
    running_.store(false, std::memory_order_release);
    if (thread_.joinable()) thread_.join();
    if (stop_hook_) stop_hook_();
}

void CpuPollingThread::publish_done(uint64_t value) {
    uint64_t cur = __atomic_load_n(&queue_->done_idx, __ATOMIC_RELAXED);
    if (value > cur) __atomic_store_n(&queue_->done_idx, value, __ATOMIC_RELEASE);
}

// Completion point for everything issued so far: once those copies finish,
// done_idx = done_value and the pending host-side flags are written.
void CpuPollingThread::push_completion(uint64_t done_value) {
    CompletionFifo& f = *fifo_;
    while (f.count == CompletionFifo::N) drain_completions(true);
    CompletionSlot& s = f.slots[f.head];
    s.fence = ce_manager_.fence();
    s.worker_job = worker_posted_;
    s.done_value = done_value;
    s.host_tiles.swap(pending_.host_tiles);
    s.host_lists.swap(pending_.host_lists);
    s.lists_done = pending_.lists_done;
    pending_.clear();
    f.head = (f.head + 1) % CompletionFifo::N;
    f.count++;
}

void CpuPollingThread::finish_slot(CompletionSlot& s) {
    if (tiled_queue_)
        for (auto& tv : s.host_tiles)
            __atomic_store_n(&tiled_queue_->tile_chunk_done[tv.first], tv.second, __ATOMIC_RELEASE);
    if (sg_queue_) {
        for (uint32_t id : s.host_lists) __atomic_store_n(&sg_queue_->d_list_done[id], 1ull, __ATOMIC_RELEASE);
        if (s.lists_done) __atomic_fetch_add(&sg_queue_->lists_completed, (uint64_t)s.lists_done, __ATOMIC_RELEASE);
    }
    s.clear();
}

// Publish every completed slot in order; with `block`, wait for the oldest.
void CpuPollingThread::drain_completions(bool block) {
    CompletionFifo& f = *fifo_;
    while (f.count > 0) {
        CompletionSlot& s = f.slots[f.tail];
        if (!ce_manager_.fence_done(s.fence)) {
            if (!block) return;
            if (ce_manager_.wait_fence(s.fence) != 0) GFD_LOG_ERROR("a copy reported an error\n");
        }
        if (s.worker_job && !worker_->done(s.worker_job)) {
            if (!block) return;
            static const uint64_t timeout_us = (uint64_t)env_size("GFD_DIRECT_TIMEOUT_MS", 10000) * 1000ull;
            if (worker_->wait(s.worker_job, timeout_us) != 0) GFD_LOG_ERROR("a worker job did not finish\n");
        }
        if (s.worker_job > worker_done_seen_) {
            worker_done_seen_ = s.worker_job;
            trace(TRACE_ZC_DONE, 0, s.worker_job);
        }
        finish_slot(s);
        publish_done(s.done_value);
        trace(TRACE_DONE, 0, s.done_value);
        f.tail = (f.tail + 1) % CompletionFifo::N;
        f.count--;
        block = false;  // only the oldest is waited for
    }
}

void CpuPollingThread::polling_loop() {
    pin_self(poller_cpu_);
    gfd_hip_set_device(device_);
    std::vector<Descriptor> batch(MAX_BATCH_SIZE);
    int n = 0;
    uint32_t or_flags = 0;
    int threshold = BATCH_THRESHOLD;
    const bool per_chunk_flush = tiled_queue_ || sg_queue_;

    auto take = [&](Descriptor* d) {
        Descriptor& b = batch[n];
        b.src_addr = d->src_addr;
        b.dst_addr = d->dst_addr;
        b.size = d->size;
        b.flags = d->flags;
        b.user_data = d->user_data;
        or_flags |= b.flags;
        __atomic_store_n(&d->sequence, 0ull, __ATOMIC_RELEASE);
        n++;
    };

    // read_idx lives in the same cache line as done_idx, which GPU waiters
    // poll over PCIe: it is published once per run of consumed descriptors
    // rather than once per descriptor, so the line is not bounced per entry.
    uint64_t read = queue_->read_idx;
    while (running_.load(std::memory_order_acquire)) {
        Descriptor* d = &queue_->entries[read % QUEUE_SIZE];
        uint64_t seq = __atomic_load_n(&d->sequence, __ATOMIC_ACQUIRE);
        if (seq == read + 1) {
            const uint64_t t0 = now_us();
            if (n == 0) {
                if (gather_) gather_->prewake();  // wake workers while the batch is read
                trace(TRACE_BATCH_FIRST, (uint32_t)(read % QUEUE_SIZE), read);
                // The batch's ranges are looked up afresh (see flush_batch),
                // now for its first entry: the runtime lookups (a few us) then
                // overlap the writing of the rest of the batch instead of
                // delaying its flush.
                ce_manager_.forget_pinned_range();
                ce_manager_.host_source_ok(reinterpret_cast<const void*>((uintptr_t)d->src_addr), d->size);
                queue_dst_lo_ = queue_dst_hi_ = 0;
                uint64_t base = 0, bytes = 0;
                if (gfd_hip_device_range(d->dst_addr, &base, &bytes)) {
                    queue_dst_lo_ = base;
                    queue_dst_hi_ = base + bytes;
                }
                batch_checked_ = true;
            }
            do {
                // The ring lines were last written by the GPU, so each is a
                // cache miss: fetch 32 descriptors ahead of the reads (16 and
                // 64 measured equal or slower at 8192 x 4 KiB and 2048 x 512 B).
                _mm_prefetch((const char*)&queue_->entries[(read + 32) % QUEUE_SIZE], _MM_HINT_T0);
                take(d);
                read++;
                if (n == 1) threshold = batch[0].size <= 2048 ? BATCH_THRESHOLD_SMALL : BATCH_THRESHOLD;
                if (n >= threshold || n >= MAX_BATCH_SIZE) break;
                if (per_chunk_flush && (or_flags & FLAG_LAST_IN_TILE)) break;
                d = &queue_->entries[read % QUEUE_SIZE];
                seq = __atomic_load_n(&d->sequence, __ATOMIC_ACQUIRE);
            } while (seq == read + 1);
            __atomic_store_n(&queue_->read_idx, read, __ATOMIC_RELEASE);
            total_queue_read_us_.fetch_add(now_us() - t0, std::memory_order_relaxed);
            const bool urgent = (or_flags & (FLAG_LAST_IN_BATCH | FLAG_URGENT | FLAG_LAST_IN_TILE)) != 0;
            if (n >= threshold || n >= MAX_BATCH_SIZE || urgent) flush_batch(batch.data(), n, or_flags);
        } else if (n > 0) {
            bool filled = false;
            for (int spin = 0; spin < 4096; spin++) {
                cpu_relax();
                if (__atomic_load_n(&d->sequence, __ATOMIC_ACQUIRE) == read + 1) {
                    filled = true;
                    break;
                }
            }
            if (!filled) {
                trace(TRACE_GAP_FLUSH, (uint32_t)n, read);
                flush_batch(batch.data(), n, or_flags);
            }
        } else if (fifo_->count > 0) {
            drain_completions(false);
            cpu_relax();
        } else {
            cpu_relax();
        }
    }

    // Drain what is already committed, then wait for every copy.
    for (;;) {
        Descriptor* d = &queue_->entries[read % QUEUE_SIZE];
        if (__atomic_load_n(&d->sequence, __ATOMIC_ACQUIRE) != read + 1) break;
        take(d);
        read++;
        __atomic_store_n(&queue_->read_idx, read, __ATOMIC_RELEASE);
        if (n >= MAX_BATCH_SIZE) flush_batch(batch.data(), n, or_flags);
    }
    flush_batch(batch.data(), n, or_flags);
    while (fifo_->count > 0) drain_completions(true);
}

void CpuPollingThread::flush_batch(Descriptor* batch, int& count, uint32_t& or_flags) {
    if (count == 0) return;
    // A source range found pinned for an earlier batch may have been freed
    // and reused since: batches look their caller-owned sources up again
    // (and device ranges too), when their first descriptor is taken in the
    // polling loop, or here.
    if (!batch_checked_) {
        ce_manager_.forget_pinned_range();
        queue_dst_lo_ = queue_dst_hi_ = 0;
    }
    batch_checked_ = false;
    const uint64_t cur_read = queue_->read_idx;
    if (trace_on_.load(std::memory_order_relaxed)) {
        uint64_t bytes = 0;
        for (int i = 0; i < count; i++) bytes += batch[i].size;
        trace(TRACE_FLUSH, (uint32_t)count, bytes);
    }
    if (sg_queue_ && (or_flags & FLAG_LAST_IN_TILE)) {
        process_batch_sg(batch, count, cur_read);
    } else if (sg_queue_) {
        // No list ends here: the batch's last list continues in a later batch.
        const uint64_t f0 = ce_manager_.fence();
        process_batch(batch, count);
        if (!sg_open_) {
            sg_open_ = true;
            sg_open_begin_ = f0;
        }
    } else if (tiled_queue_) {
        process_batch_tiled(batch, count, cur_read);
    } else {
        process_batch(batch, count);
    }
    trace(TRACE_ISSUED, 0, ce_manager_.fence());
    push_completion(cur_read);
    drain_completions(false);
    count = 0;
    or_flags = 0;
}

// One copy per maximal run that is contiguous in both src and dst.
void CpuPollingThread::copy_runs(const SGEntry* e, int count) {
    std::vector<SGEntry>& runs = run_scratch_;
    runs.clear();
    int i = 0;
    while (i < count) {
        SGEntry r = e[i];
        int j = i + 1;
        while (j < count && e[j].dst == r.dst + r.size && (const char*)e[j].src == (const char*)r.src + r.size) {
            r.size += e[j].size;
            j++;
        }
        runs.push_back(r);
        i = j;
    }
    if (ce_manager_.submit_scatter_gather(runs.data(), (int)runs.size()) != 0)
        GFD_LOG_ERROR("copy submission failed\n");
    coalesced_entries_.fetch_add(runs.size(), std::memory_order_relaxed);
}

// Gather a dst-contiguous list through the next staging buffer; false if it
// does not fit (the caller then copies runs directly).
void CpuPollingThread::trace_gather_run() {
    if (!gather_ || !trace_on_.load(std::memory_order_relaxed)) return;
    const GatherEngine::RunTimes rt = gather_->last_run();
    trace_at(rt.entry, TRACE_GATHER_ENTRY, 0, 0);
    trace_at(rt.idle, TRACE_GATHER_IDLE, 0, 0);
    trace_at(rt.built, TRACE_GATHER_BUILT, 0, 0);
    trace_at(rt.published, TRACE_GATHER_PUBLISHED, (uint32_t)rt.sleepers, 0);
    trace_at(rt.first_slice, TRACE_GATHER_FIRST_SLICE, (uint32_t)rt.copiers, 0);
}

bool CpuPollingThread::gather_through_staging(const SGEntry* e, int count, size_t total, const DstRun* runs,
                                              int nruns, int uniform_hint) {
    if (num_staging_bufs_ == 0 || total > staging_buffer_size_ || !gather_) return false;
    const int cur = staging_cur_;
    const uint64_t t0 = now_us();
    if (ce_manager_.wait_fence(staging_fence_[cur]) != 0) GFD_LOG_ERROR("staging copy reported an error\n");
    const uint64_t t1 = now_us();
    ChunkCtx ctx{this, &ce_manager_, e[0].dst, staging_bufs_[cur], ce_manager_.num_channels(), 0};
    RunCopyCtx rctx{this, &ce_manager_, staging_bufs_[cur], runs, nruns, 0, ce_manager_.num_channels(), 0, 0};
    {
        std::lock_guard<std::mutex> lock(gather_mutex_);
        if (runs)
            gather_->run(e, count, total, staging_bufs_[cur], direct_chunk_bytes_, run_copy_chunk, &rctx,
                         uniform_hint);
        else
            gather_->run(e, count, total, staging_bufs_[cur], direct_chunk_bytes_, issue_chunk, &ctx, uniform_hint);
        trace_gather_run();
    }
    if (rctx.err && !ctx.err) ctx.err = rctx.err;
    const uint64_t t2 = now_us();
    staging_fence_[cur] = ce_manager_.fence();
    staging_cur_ = (cur + 1) % num_staging_bufs_;
    total_dma_wait_us_.fetch_add(t1 - t0, std::memory_order_relaxed);
    total_gather_us_.fetch_add(t2 - t1, std::memory_order_relaxed);
    staging_batches_.fetch_add(1, std::memory_order_relaxed);
    coalesced_entries_.fetch_add(count, std::memory_order_relaxed);
    if (ctx.err) GFD_LOG_ERROR("staging copy submission failed (%d)\n", ctx.err);
    return true;
}

// Route one list: contiguous on both sides -> one copy; dst contiguous ->
// staged gather; up to kMaxRunCopies destination runs -> staged gather with
// one copy per run piece; otherwise one copy per run contiguous on both
// sides.  (No kernel is launched here: Queue-path consumers spin on the GPU,
// and a kernel could queue behind them on a shared hardware queue.)
void CpuPollingThread::submit_list(const SGEntry* e, int count, size_t total) {
    bool dst_contig = true, src_contig = true, uniform = true;
    for (int i = 1; i < count; i++) {
        dst_contig &= e[i].dst == e[i - 1].dst + e[i - 1].size;
        src_contig &= (const char*)e[i].src == (const char*)e[i - 1].src + e[i - 1].size;
        uniform &= e[i].size == e[0].size;
    }
    submit_list(e, count, total, dst_contig, src_contig, uniform);
}

void CpuPollingThread::submit_list(const SGEntry* e, int count, size_t total, bool dst_contig, bool src_contig,
                                   bool uniform) {
    const uint64_t t0 = now_us();
    if (queue_worker_copy(e, count, total)) {
        coalesced_entries_.fetch_add((uint64_t)count, std::memory_order_relaxed);
    } else if (count == 1 || (dst_contig && src_contig)) {
        SGEntry one{e[0].dst, e[0].src, total};
        ce_manager_.submit_scatter_gather(&one, 1);
        coalesced_entries_.fetch_add(1, std::memory_order_relaxed);
    } else if (dst_contig) {
        if (!gather_through_staging(e, count, total, nullptr, 0, uniform ? 1 : 0)) copy_runs(e, count);
    } else {
        const int nr = dst_runs(e, count, kMaxRunCopies, queue_runs_);
        if (!(nr <= kMaxRunCopies &&
              gather_through_staging(e, count, total, queue_runs_.data(), nr, uniform ? 1 : 0)))
            copy_runs(e, count);
    }
    total_dma_submit_us_.fetch_add(now_us() - t0, std::memory_order_relaxed);
}

// The previous batch's gather workers still hold this array's lines in their
// caches: plain stores would take each line back one by one (12.6 us for
// 4096 entries against 5 us unshared).  Streaming stores skip those reads,
// and the route's contiguity tests are made here from the poller's own copy.
bool CpuPollingThread::process_batch(Descriptor* batch, int count) {
    std::vector<SGEntry>& sg = sg_scratch_;
    sg.resize(count);
    size_t total = 0;
    bool dst_contig = true, src_contig = true, uniform = true;
    uint64_t dst_end = batch[0].dst_addr, src_end = batch[0].src_addr;
    const uint64_t size0 = batch[0].size;
    for (int i = 0; i < count; i++) {
        const uint64_t d = batch[i].dst_addr, s = batch[i].src_addr, n = batch[i].size;
        dst_contig &= d == dst_end;
        src_contig &= s == src_end;
        uniform &= n == size0;
        dst_end = d + n;
        src_end = s + n;
        total += n;
        long long* out = reinterpret_cast<long long*>(&sg[i]);
        _mm_stream_si64(out, (long long)d);
        _mm_stream_si64(out + 1, (long long)s);
        _mm_stream_si64(out + 2, (long long)n);
    }
    _mm_sfence();
    total_bytes_copied_.fetch_add(total, std::memory_order_relaxed);
    descriptors_processed_.fetch_add(count, std::memory_order_relaxed);
    batches_submitted_.fetch_add(1, std::memory_order_relaxed);
    // The workers gather from this array: telling run() the list is uniform
    // spares it a pass over entries just written with streaming stores.
    submit_list(sg.data(), count, total, dst_contig, src_contig, uniform);
    return true;
}

// 8-byte store of `value` into HBM at `dst`, ordered on the copy engines after
// every copy with fence >= after_begin issued so far.
void CpuPollingThread::signal_device_u64(uint64_t* dst, uint64_t value, uint64_t after_begin) {
    const int slot = signal_next_;
    signal_next_ = (signal_next_ + 1) % SIGNAL_SLOTS;
    ce_manager_.wait_fence(signal_fence_[slot]);  // previous use of this value slot has finished
    signal_values_[slot] = value;
    const uint64_t end = ce_manager_.fence();
    // Chained after the previous flag write as well as after its own batch's
    // copies: two progress writes to one tile issued back to back could
    // otherwise land out of order on different engines and leave the older,
    // smaller count in place.
    if (ce_manager_.submit_after((DevicePtr)(uintptr_t)dst, &signal_values_[slot], sizeof(uint64_t), after_begin,
                                 end, last_signal_copy_) != 0)
        GFD_LOG_ERROR("flag write submission failed\n");
    else
        last_signal_copy_ = end;  // the copy just issued got fence number `end`
    signal_fence_[slot] = ce_manager_.fence();
}

// Tiled mode: entries carry tile_id in user_data >> 32.  Every tile touched by
// the batch gets its cumulative progress written after the batch's copies.
void CpuPollingThread::process_batch_tiled(Descriptor* batch, int count, uint64_t cur_read) {
    (void)cur_read;
    const uint64_t f0 = ce_manager_.fence();
    process_batch(batch, count);
    std::vector<uint32_t>& touched = tile_scratch_;
    touched.clear();
    for (int i = 0; i < count; i++) {
        const uint32_t tid = (uint32_t)(batch[i].user_data >> 32);
        if (tid >= (uint32_t)MAX_TILES) continue;
        if (tile_progress_[tid]++ == tile_marked_[tid]) touched.push_back(tid);
    }
    if (tile_done_on_device_ < 0)
        tile_done_on_device_ = tiled_queue_->d_tile_chunk_done ? gfd_hip_pointer_is_device(tiled_queue_->d_tile_chunk_done) : 0;
    for (uint32_t tid : touched) {
        tile_marked_[tid] = tile_progress_[tid];
        if (tiled_queue_->d_tile_chunk_done && tile_done_on_device_)
            signal_device_u64(tiled_queue_->d_tile_chunk_done + tid, tile_progress_[tid], f0);
        else
            pending_.host_tiles.emplace_back(tid, tile_progress_[tid]);
    }
}

// SG mode: entries carry list_id in user_data >> 32; each list is copied on
// its own and d_list_done[list_id] = 1 once its copies have finished.
void CpuPollingThread::process_batch_sg(Descriptor* batch, int count, uint64_t cur_read) {
    (void)cur_read;
    if (list_done_on_device_ < 0)
        list_done_on_device_ = sg_queue_->d_list_done ? gfd_hip_pointer_is_device(sg_queue_->d_list_done) : 0;
    std::vector<SGEntry> list;
    int i = 0;
    while (i < count) {
        const uint32_t list_id = (uint32_t)(batch[i].user_data >> 32);
        int j = i;
        size_t total = 0;
        list.clear();
        while (j < count && (uint32_t)(batch[j].user_data >> 32) == list_id) {
            list.push_back(SGEntry{batch[j].dst_addr, (const void*)(uintptr_t)batch[j].src_addr, batch[j].size});
            total += batch[j].size;
            j++;
        }
        const uint64_t f0 = ce_manager_.fence();
        // The batch's first run may finish a list opened in earlier batches:
        // its flag then waits for those batches' copies too.
        const bool continues = i == 0 && sg_open_;
        const uint64_t begin = continues ? sg_open_begin_ : f0;
        submit_list(list.data(), (int)list.size(), total);
        total_bytes_copied_.fetch_add(total, std::memory_order_relaxed);
        descriptors_processed_.fetch_add(j - i, std::memory_order_relaxed);
        batches_submitted_.fetch_add(1, std::memory_order_relaxed);
        const bool list_end = (batch[j - 1].flags & FLAG_LAST_IN_TILE) != 0;
        if (list_end && sg_queue_->d_list_done && list_id < (uint32_t)MAX_SG_LISTS) {
            if (list_done_on_device_)
                signal_device_u64(sg_queue_->d_list_done + list_id, 1, begin);
            else
                pending_.host_lists.push_back(list_id);
        }
        if (list_end) {
            pending_.lists_done++;
            sg_open_ = false;
        } else {
            // Only the batch's last run can leave its list open.
            if (!continues) sg_open_begin_ = f0;
            sg_open_ = true;
        }
        i = j;
    }
}

}  // namespace gfd
