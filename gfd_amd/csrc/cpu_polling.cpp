// CpuPollingThread: lifecycle, resources and the descriptor-ring poller
// (declaration: include/gfd/cpu_polling.h).
//
// Reference behaviour kept (src/cpu_polling.cpp:37-490,
// src/batch_processor.cpp:448-723):
//   * a descriptor is consumed when sequence == read_idx + 1 (acquire); the
//     poller zeroes sequence (release) and advances read_idx;
//   * batches close at BATCH_THRESHOLD entries (BATCH_THRESHOLD_SMALL when the
//     first entry is <= 2 KB), at MAX_BATCH_SIZE, on LAST_IN_BATCH / URGENT /
//     LAST_IN_TILE, or after a 4096-pause gap with no new descriptor;
//   * a dst-contiguous, equal-size, src-scattered batch is gathered into the
//     next of NUM_STAGING_BUFS rotating pinned buffers and copied as one range;
//   * done_idx only ever moves forward and only past slots whose copies have
//     completed.
// MI355X design differences:
//   * done_idx is advanced per batch as soon as that batch's copies finish (a
//     FIFO of completion events recorded on a signal stream that waits on all
//     copy channels), not only when the ring goes idle;
//   * the batch gather is pipelined: staging chunks are copied as soon as the
//     worker pool finishes them;
//   * per-list / per-tile signals are stream-ordered 8-byte writes into HBM
//     queued behind the data copies (hipStreamWriteValue64).
#include "gfd/cpu_polling.h"

#include <immintrin.h>
#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <vector>

#include "gather_engine.h"
#include "gfd/pcie_topology.h"
#include "gfd/sg_task_queue.h"
#include "gfd/staging_pool.h"
#include "poller_internal.h"

namespace gfd {

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
    fifo_ = new CompletionFifo();
}

CpuPollingThread::~CpuPollingThread() {
    stop();
    delete gather_;
    gather_ = nullptr;
    gfd_hip_set_device(device_);
    ce_manager_.wait_completion();
    direct_ce_manager_.wait_completion();
    if (signal_stream_) {
        gfd_hip_stream_synchronize(signal_stream_);
        gfd_hip_stream_destroy(signal_stream_);
        signal_stream_ = nullptr;
    }
    for (int b = 0; b < NUM_STAGING_BUFS; b++) {
        if (staging_events_[b]) gfd_hip_event_destroy(staging_events_[b]);
        staging_events_[b] = nullptr;
    }
    if (fifo_) {
        for (auto& s : fifo_->slots)
            if (s.event) gfd_hip_event_destroy(s.event);
        delete fifo_;
        fifo_ = nullptr;
    }
    if (staging_pool_set_ >= 0) {
        StagingPool::instance().release_buffers(staging_pool_set_);
        staging_pool_set_ = -1;
    } else if (staging_owned_) {
        for (int b = 0; b < NUM_STAGING_BUFS; b++) StagingPool::free_pinned(staging_bufs_[b]);
    }
    for (int b = 0; b < NUM_STAGING_BUFS; b++) staging_bufs_[b] = nullptr;
    StagingPool::free_pinned(direct_staging_);
    direct_staging_ = nullptr;
    ce_manager_.shutdown();
    direct_ce_manager_.shutdown();
}

int CpuPollingThread::num_gather_workers() const { return gather_ ? gather_->num_workers() : 0; }

void CpuPollingThread::set_gather_slice_bytes(size_t b) {
    slice_bytes_ = b;
    if (gather_) gather_->set_slice_bytes(b);
}

bool CpuPollingThread::choose_cpus() {
    if (cpus_chosen_) return true;
    GpuTopology topo = discover_gpu_topology(device_);
    if (numa_node_ < 0) numa_node_ = topo.numa_node;
    int cap = (int)env_size("GFD_NUM_GATHER_WORKERS", MAX_GATHER_WORKERS);
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
    GFD_LOG_INFO("gather workers: %d (poller CPU %d, NUMA %d)\n", gather_->num_workers(), poller_cpu_,
                 numa_node_);
    return true;
}

bool CpuPollingThread::init_copy_engine() {
    if (!use_ce_) {
        GFD_LOG_ERROR("use_ce=false is not supported: copies always use the SDMA channels\n");
        return false;
    }
    if (gfd_hip_set_device(device_) != 0) return false;
    choose_cpus();
    if (ce_manager_.init(device_, num_ce_channels_) != 0) {
        GFD_LOG_ERROR("copy engine init failed\n");
        return false;
    }
    if (!signal_stream_ && gfd_hip_stream_create(&signal_stream_) != 0) {
        GFD_LOG_ERROR("signal stream creation failed\n");
        return false;
    }
    for (auto& s : fifo_->slots)
        if (!s.event && gfd_hip_event_create(&s.event, 0) != 0) return false;

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
    for (int b = 0; b < got; b++) {
        if (!staging_events_[b] && gfd_hip_event_create(&staging_events_[b], 0) != 0) return false;
        staging_event_pending_[b] = false;
    }
    GFD_LOG_INFO("queue staging: %d x %zu bytes (NUMA %d)\n", got, staging_buffer_size_, numa_node_);
    return start_workers();
}

void CpuPollingThread::start() {
    if (running_.load(std::memory_order_acquire)) return;
    if (!queue_) {
        GFD_LOG_ERROR("start(): no descriptor queue\n");
        return;
    }
    running_.store(true, std::memory_order_release);
    thread_ = std::thread(&CpuPollingThread::polling_loop, this);
}

void CpuPollingThread::stop() {
    running_.store(false, std::memory_order_release);
    if (thread_.joinable()) thread_.join();
}

void CpuPollingThread::publish_done(uint64_t value) {
    uint64_t cur = __atomic_load_n(&queue_->done_idx, __ATOMIC_RELAXED);
    if (value > cur) __atomic_store_n(&queue_->done_idx, value, __ATOMIC_RELEASE);
}

// Record a completion point for everything submitted so far on the copy
// channels; it publishes done_idx = done_value (and the tiles / lists noted in
// the slot) once the GPU passes it.
void CpuPollingThread::push_completion(uint64_t done_value) {
    CompletionFifo& f = *fifo_;
    while (f.count == CompletionFifo::N) drain_completions(true);
    CompletionSlot& s = f.slots[f.head];
    if (ce_manager_.make_stream_wait_on_all(signal_stream_) != 0 ||
        gfd_hip_event_record(s.event, signal_stream_) != 0) {
        // Could not record: wait for everything and publish directly.
        ce_manager_.wait_completion();
        gfd_hip_stream_synchronize(signal_stream_);
        finish_slot(s_pending_);
        publish_done(done_value);
        s_pending_.clear();
        return;
    }
    s.done_value = done_value;
    s.host_tiles.swap(s_pending_.host_tiles);
    s.lists_done = s_pending_.lists_done;
    s_pending_.clear();
    f.head = (f.head + 1) % CompletionFifo::N;
    f.count++;
}

void CpuPollingThread::finish_slot(CompletionSlot& s) {
    if (tiled_queue_)
        for (auto& tv : s.host_tiles)
            __atomic_store_n(&tiled_queue_->tile_chunk_done[tv.first], tv.second, __ATOMIC_RELEASE);
    s.host_tiles.clear();
    if (sg_queue_ && s.lists_done)
        __atomic_fetch_add(&sg_queue_->lists_completed, (uint64_t)s.lists_done, __ATOMIC_RELEASE);
    s.lists_done = 0;
}

// Publish every completed slot in order; with `block`, wait for the oldest.
void CpuPollingThread::drain_completions(bool block) {
    CompletionFifo& f = *fifo_;
    while (f.count > 0) {
        CompletionSlot& s = f.slots[f.tail];
        int q = gfd_hip_event_query(s.event);
        if (q == 1) {
            if (!block) return;
            while ((q = gfd_hip_event_query(s.event)) == 1) cpu_relax();
        }
        if (q != 0) GFD_LOG_ERROR("completion event error %d\n", q);
        finish_slot(s);
        publish_done(s.done_value);
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

    while (running_.load(std::memory_order_acquire)) {
        uint64_t read = queue_->read_idx;
        Descriptor* d = &queue_->entries[read % QUEUE_SIZE];
        uint64_t seq = __atomic_load_n(&d->sequence, __ATOMIC_ACQUIRE);
        if (seq == read + 1) {
            do {
                take(d);
                read++;
                __atomic_store_n(&queue_->read_idx, read, __ATOMIC_RELEASE);
                if (n == 1) threshold = batch[0].size <= 2048 ? BATCH_THRESHOLD_SMALL : BATCH_THRESHOLD;
                if (n >= threshold || n >= MAX_BATCH_SIZE) break;
                if (per_chunk_flush && (or_flags & FLAG_LAST_IN_TILE)) break;
                d = &queue_->entries[read % QUEUE_SIZE];
                seq = __atomic_load_n(&d->sequence, __ATOMIC_ACQUIRE);
            } while (seq == read + 1);
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
            if (!filled) flush_batch(batch.data(), n, or_flags);
        } else if (fifo_->count > 0) {
            drain_completions(false);
            cpu_relax();
        } else {
            cpu_relax();
        }
    }

    // Drain what is already committed, then wait for every copy.
    for (;;) {
        uint64_t read = queue_->read_idx;
        Descriptor* d = &queue_->entries[read % QUEUE_SIZE];
        if (__atomic_load_n(&d->sequence, __ATOMIC_ACQUIRE) != read + 1) break;
        take(d);
        __atomic_store_n(&queue_->read_idx, read + 1, __ATOMIC_RELEASE);
        if (n >= MAX_BATCH_SIZE) flush_batch(batch.data(), n, or_flags);
    }
    flush_batch(batch.data(), n, or_flags);
    while (fifo_->count > 0) drain_completions(true);
}

void CpuPollingThread::flush_batch(Descriptor* batch, int& count, uint32_t& or_flags) {
    if (count == 0) return;
    const uint64_t cur_read = queue_->read_idx;
    if (sg_queue_ && (or_flags & FLAG_LAST_IN_TILE)) {
        process_batch_sg(batch, count, cur_read);
    } else if (tiled_queue_) {
        process_batch_tiled(batch, count, cur_read);
    } else {
        process_batch(batch, count);
    }
    push_completion(cur_read);
    drain_completions(false);
    count = 0;
    or_flags = 0;
}

namespace {

struct ChunkCtx {
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
}

}  // namespace

// Copy a run list: maximal runs contiguous in both src and dst become one copy.
void CpuPollingThread::copy_runs(const SGEntry* e, int count) {
    int i = 0;
    std::vector<SGEntry>& runs = run_scratch_;
    runs.clear();
    while (i < count) {
        SGEntry r = e[i];
        int j = i + 1;
        while (j < count && e[j].dst == r.dst + r.size &&
               (const char*)e[j].src == (const char*)r.src + r.size) {
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

// Gather a dst-contiguous list through the next staging buffer; true if done.
bool CpuPollingThread::gather_through_staging(const SGEntry* e, int count, size_t total) {
    if (num_staging_bufs_ == 0 || total > staging_buffer_size_ || !gather_) return false;
    const int cur = staging_cur_;
    uint64_t t0 = now_us();
    if (staging_event_pending_[cur]) {
        gfd_hip_event_synchronize(staging_events_[cur]);
        staging_event_pending_[cur] = false;
    }
    uint64_t t1 = now_us();
    ChunkCtx ctx{&ce_manager_, e[0].dst, staging_bufs_[cur], ce_manager_.num_channels(), 0};
    {
        std::lock_guard<std::mutex> lock(gather_mutex_);
        gather_->run(e, count, total, staging_bufs_[cur], direct_chunk_bytes_, issue_chunk, &ctx);
    }
    uint64_t t2 = now_us();
    // The staging buffer is free again once every channel has passed this point.
    ce_manager_.make_stream_wait_on_all(signal_stream_);
    gfd_hip_event_record(staging_events_[cur], signal_stream_);
    staging_event_pending_[cur] = true;
    staging_cur_ = (cur + 1) % num_staging_bufs_;
    total_dma_wait_us_.fetch_add(t1 - t0, std::memory_order_relaxed);
    total_gather_us_.fetch_add(t2 - t1, std::memory_order_relaxed);
    staging_batches_.fetch_add(1, std::memory_order_relaxed);
    coalesced_entries_.fetch_add(count, std::memory_order_relaxed);
    if (ctx.err) GFD_LOG_ERROR("staging copy submission failed (%d)\n", ctx.err);
    return true;
}

bool CpuPollingThread::process_batch(Descriptor* batch, int count) {
    std::vector<SGEntry>& sg = sg_scratch_;
    sg.resize(count);
    size_t total = 0;
    for (int i = 0; i < count; i++) {
        sg[i].dst = batch[i].dst_addr;
        sg[i].src = (const void*)(uintptr_t)batch[i].src_addr;
        sg[i].size = batch[i].size;
        total += batch[i].size;
    }
    total_bytes_copied_.fetch_add(total, std::memory_order_relaxed);
    descriptors_processed_.fetch_add(count, std::memory_order_relaxed);
    batches_submitted_.fetch_add(1, std::memory_order_relaxed);
    submit_list(sg.data(), count, total);
    return true;
}

// Route one list: contiguous on both sides -> one copy; dst contiguous ->
// staged gather; otherwise coalesced runs.
void CpuPollingThread::submit_list(const SGEntry* e, int count, size_t total) {
    uint64_t t0 = now_us();
    bool dst_contig = true, src_contig = true;
    for (int i = 1; i < count; i++) {
        if (e[i].dst != e[i - 1].dst + e[i - 1].size) dst_contig = false;
        if ((const char*)e[i].src != (const char*)e[i - 1].src + e[i - 1].size) src_contig = false;
        if (!dst_contig && !src_contig) break;
    }
    if (count == 1 || (dst_contig && src_contig)) {
        SGEntry one{e[0].dst, e[0].src, total};
        ce_manager_.submit_scatter_gather(&one, 1);
        coalesced_entries_.fetch_add(1, std::memory_order_relaxed);
    } else if (!(dst_contig && gather_through_staging(e, count, total))) {
        copy_runs(e, count);
    }
    total_dma_submit_us_.fetch_add(now_us() - t0, std::memory_order_relaxed);
}

// Tiled mode: entries carry tile_id in user_data >> 32.  Every tile's
// cumulative progress is written after this batch's copies complete.
void CpuPollingThread::process_batch_tiled(Descriptor* batch, int count, uint64_t cur_read) {
    (void)cur_read;
    process_batch(batch, count);
    std::vector<uint32_t>& touched = tile_scratch_;
    touched.clear();
    for (int i = 0; i < count; i++) {
        uint32_t tid = (uint32_t)(batch[i].user_data >> 32);
        if (tid >= (uint32_t)MAX_TILES) continue;
        if (tile_progress_[tid]++ == tile_marked_[tid]) touched.push_back(tid);
    }
    for (uint32_t tid : touched) {
        tile_marked_[tid] = tile_progress_[tid];
        if (tiled_queue_->d_tile_chunk_done) {
            ce_manager_.make_stream_wait_on_all(signal_stream_);
            gfd_hip_stream_write_u64(signal_stream_, (uint64_t)(uintptr_t)(tiled_queue_->d_tile_chunk_done + tid),
                                     tile_progress_[tid]);
        } else {
            s_pending_.host_tiles.emplace_back(tid, tile_progress_[tid]);
        }
    }
}

// SG mode: entries carry list_id in user_data >> 32; each list is copied on
// its own and d_list_done[list_id] = 1 is written behind its copies.
void CpuPollingThread::process_batch_sg(Descriptor* batch, int count, uint64_t cur_read) {
    (void)cur_read;
    std::vector<SGEntry>& sg = sg_scratch_;
    int i = 0;
    while (i < count) {
        const uint32_t list_id = (uint32_t)(batch[i].user_data >> 32);
        int j = i;
        size_t total = 0;
        sg.clear();
        while (j < count && (uint32_t)(batch[j].user_data >> 32) == list_id) {
            sg.push_back(SGEntry{batch[j].dst_addr, (const void*)(uintptr_t)batch[j].src_addr, batch[j].size});
            total += batch[j].size;
            j++;
        }
        submit_list(sg.data(), (int)sg.size(), total);
        total_bytes_copied_.fetch_add(total, std::memory_order_relaxed);
        descriptors_processed_.fetch_add(j - i, std::memory_order_relaxed);
        batches_submitted_.fetch_add(1, std::memory_order_relaxed);
        const bool list_end = (batch[j - 1].flags & FLAG_LAST_IN_TILE) != 0;
        if (list_end && sg_queue_ && sg_queue_->d_list_done && list_id < (uint32_t)MAX_SG_LISTS) {
            ce_manager_.make_stream_wait_on_all(signal_stream_);
            gfd_hip_stream_write_u64(signal_stream_, (uint64_t)(uintptr_t)(sg_queue_->d_list_done + list_id), 1);
        }
        if (list_end) s_pending_.lists_done++;
        i = j;
    }
}

}  // namespace gfd
