#pragma once
// CpuPollingThread: the host side of GFD.  Public interface as in
// include/gfd/cpu_polling.h:19-84 of the reference:
//   * submit_direct()  — the CPU hands an SG list straight in ("GFD Direct");
//   * start()/stop()   — a pinned thread polls the descriptor ring that GPU
//                        kernels fill ("GFD Queue"), batches contiguous runs and
//                        signals completion through done_idx and per-tile /
//                        per-list flags.
// Both gather scattered host tokens into pinned staging memory with a pool of
// worker threads and stream the staging to HBM over SDMA engines.
//
// Threading: init_copy_engine()/init_direct_ce() must run on a thread that can
// use the GPU; the polling thread makes the device current itself.
// submit_direct() may run concurrently with the polling thread: the gather
// workers are shared under a mutex and each path has its own staging buffers
// and its own copy channels.
#include <atomic>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

#include "gfd/copy_engine.h"
#include "gfd/tiled_queue.h"

namespace gfd {

// Upper bound on gather worker threads (not counting the calling thread).
constexpr int MAX_GATHER_WORKERS = 15;
// Worker count the reference used when no core range was given.
constexpr int NUM_GATHER_WORKERS = 7;

struct SGTaskQueue;
class GatherEngine;
class ZcWorker;

class CpuPollingThread {
public:
    // queue:          descriptor ring in fine-grained host memory (may be null
    //                 for direct-only use)
    // gpu_base:       base of the HBM destination region (informational)
    // cpu_base/total_cpu_size: the host source region; staging buffers are
    //                 sized to total_cpu_size
    // use_ce:         false = no copy engines (kept for API compatibility;
    //                 init_copy_engine() then fails)
    // numa_node:      host node for staging and workers; -1 = the GPU's node
    // core_offset:    kept for API compatibility (ignored: CPUs are chosen from
    //                 the node's CPU list and the process affinity mask)
    // num_ce_channels: copy channels per manager (0 = default)
    // exclusive_core_base/count: explicit CPU range for poller + workers
    CpuPollingThread(DescriptorQueue* queue, void* gpu_base, void* cpu_base,
                     size_t total_cpu_size, bool use_ce = true, int numa_node = 0,
                     int core_offset = 0, int num_ce_channels = 0,
                     int exclusive_core_base = -1, int exclusive_core_count = 0);
    ~CpuPollingThread();
    CpuPollingThread(const CpuPollingThread&) = delete;
    CpuPollingThread& operator=(const CpuPollingThread&) = delete;

    // Copy channels, staging buffers, gather workers.
    bool init_copy_engine();

    // Separate copy channels and staging for submit_direct().
    bool init_direct_ce();

    // Gather `count` entries into HBM and block until they have landed.
    // Returns the wall time in microseconds, or -1 on error.
    // Paths (src/direct_submit.cpp:37-145):
    //   src and dst contiguous      -> one copy split over the channels
    //   dst contiguous, src scattered, total <= staging
    //                               -> pipelined gather: the workers fill
    //                                  staging chunk by chunk and each finished
    //                                  chunk is copied at once on the next channel
    //   otherwise                   -> one copy per maximal contiguous run
    double submit_direct(const SGEntry* entries, int count);

    void set_tiled_queue(TiledQueue* tq) { tiled_queue_ = tq; }
    // SG mode is switched off in the product library: start() logs an error
    // and does not start while an SG task queue is set (is_running() then
    // stays false).
    void set_sg_task_queue(SGTaskQueue* sq) { sg_queue_ = sq; }

    void start();
    void stop();
    // True between a start() that launched the polling thread and stop().
    bool is_running() const { return running_.load(std::memory_order_acquire); }

    uint64_t get_descriptors_processed() const { return descriptors_processed_.load(std::memory_order_relaxed); }
    uint64_t get_batches_submitted() const { return batches_submitted_.load(std::memory_order_relaxed); }
    uint64_t get_coalesced_entries() const { return coalesced_entries_.load(std::memory_order_relaxed); }
    uint64_t get_staging_batches() const { return staging_batches_.load(std::memory_order_relaxed); }
    double get_total_bytes_copied() const { return (double)total_bytes_copied_.load(std::memory_order_relaxed); }
    const CopyEngineManager& get_ce_manager() const { return ce_manager_; }
    bool is_ce_mode() const { return use_ce_; }
    uint64_t get_gather_us() const { return total_gather_us_.load(std::memory_order_relaxed); }
    uint64_t get_dma_wait_us() const { return total_dma_wait_us_.load(std::memory_order_relaxed); }
    uint64_t get_dma_submit_us() const { return total_dma_submit_us_.load(std::memory_order_relaxed); }
    uint64_t get_queue_read_us() const { return total_queue_read_us_.load(std::memory_order_relaxed); }

    // Only between runs (the polling thread stopped or idle).
    void reset_stats() {
        descriptors_processed_.store(0, std::memory_order_relaxed);
        batches_submitted_.store(0, std::memory_order_relaxed);
        coalesced_entries_.store(0, std::memory_order_relaxed);
        staging_batches_.store(0, std::memory_order_relaxed);
        total_bytes_copied_.store(0, std::memory_order_relaxed);
        total_gather_us_.store(0, std::memory_order_relaxed);
        total_dma_wait_us_.store(0, std::memory_order_relaxed);
        total_dma_submit_us_.store(0, std::memory_order_relaxed);
        total_queue_read_us_.store(0, std::memory_order_relaxed);
        std::memset(tile_progress_, 0, sizeof(tile_progress_));
        std::memset(tile_marked_, 0, sizeof(tile_marked_));
    }

    // ---- MI355X additions -------------------------------------------------
    // Data moved by the transfer waves of the session that owns this poller
    // (sessions copy with their own waves, not through the poller): the
    // session adds what each launch landed, so the stats getters above count
    // it (entries as descriptors, lists or tiles as batches, and bytes).
    void add_device_landed(uint64_t entries, uint64_t bytes, uint64_t batches) {
        descriptors_processed_.fetch_add(entries, std::memory_order_relaxed);
        total_bytes_copied_.fetch_add(bytes, std::memory_order_relaxed);
        batches_submitted_.fetch_add(batches, std::memory_order_relaxed);
    }
    // Called at the end of every stop() (set by an owning session, which then
    // takes in the results of a kernel the caller launched itself between
    // start() and stop(); an empty function clears it).
    void set_stop_hook(std::function<void()> hook) { stop_hook_ = std::move(hook); }
    int num_gather_workers() const;
    const std::vector<int>& worker_cpus() const { return worker_cpus_; }
    int poller_cpu() const { return poller_cpu_; }
    int numa_node() const { return numa_node_; }
    int device() const { return device_; }
    const CopyEngineManager& get_direct_ce_manager() const { return direct_ce_manager_; }
    // Destination-contiguous lists of at most this many bytes whose sources
    // are pinned host memory go through the zero-copy gather kernel instead
    // of the staged SDMA copies (0 = never; GFD_DIRECT_ZC_MAX_BYTES).  Below
    // a few MiB the copy engines' fixed start-up latency dominates.
    void set_direct_zero_copy_max_bytes(size_t b) { direct_zc_max_bytes_ = b; }
    size_t direct_zero_copy_max_bytes() const { return direct_zc_max_bytes_; }
    // Lists of at most this many bytes take the staged SDMA route even when
    // the zero-copy kernel could move them: at these sizes a copy-engine copy
    // starts sooner than a kernel launch (GFD_DIRECT_ZC_MIN_BYTES; 64 KiB).
    void set_direct_zero_copy_min_bytes(size_t b) { direct_zc_min_bytes_ = b; }
    size_t direct_zero_copy_min_bytes() const { return direct_zc_min_bytes_; }
    // Larger destination-contiguous lists with pinned sources: the zero-copy
    // kernel moves the first entries, up to this many bytes, while the gather
    // workers stage the rest for the copy engines, so the host link carries
    // data before the first staged chunk is ready (0 = off;
    // GFD_DIRECT_ZC_HEAD_BYTES; needs the zero-copy route enabled).
    void set_direct_zero_copy_head_bytes(size_t b) { direct_zc_head_bytes_ = b; }
    size_t direct_zero_copy_head_bytes() const { return direct_zc_head_bytes_; }
    // The persistent zero-copy worker (off by default; GFD_ZC_WORKER=1 turns
    // it on for new pollers): a grid of 64 waves that stays resident on an
    // AQL queue of this poller's own and copies a list when the host rings
    // its doorbell, ending itself after GFD_ZC_WORKER_IDLE_MS (100 ms)
    // without a job.  While it is on, submit_direct sends every destination-
    // contiguous list of at most direct_zero_copy_max_bytes() with pinned
    // sources to it (short ones included), and the Queue path sends batches
    // of at most worker_queue_max_bytes() with pinned sources and device
    // destinations to it instead of staging them for the copy engines.
    // Returns 0, or nonzero if the worker cannot be set up (it then stays
    // off).  Not while the polling thread runs.
    int set_zero_copy_worker(bool on);
    bool zero_copy_worker() const { return worker_ != nullptr; }
    // Jobs the worker ran and grids dispatched for them (0 when off).
    uint64_t zero_copy_worker_jobs() const;
    uint64_t zero_copy_worker_launches() const;
    // The worker's device timeline of its latest jobs (see ZcWorker::
    // read_timeline): up to max_jobs records of 8 words, newest first.
    int zero_copy_worker_timeline(uint64_t* out, int max_jobs);
    void set_worker_queue_max_bytes(size_t b) { worker_queue_max_bytes_ = b; }
    size_t worker_queue_max_bytes() const { return worker_queue_max_bytes_; }
    // Chunk size of the pipelined gather (payload bytes per copy).
    void set_direct_chunk_bytes(size_t b) { direct_chunk_bytes_ = b ? b : 1; }
    size_t direct_chunk_bytes() const { return direct_chunk_bytes_; }
    // Gather slice size (bytes one thread copies per work item).
    void set_gather_slice_bytes(size_t b);
    size_t gather_slice_bytes() const { return slice_bytes_; }
    size_t staging_buffer_size() const { return staging_buffer_size_; }
    int num_staging_buffers() const { return num_staging_bufs_; }
    // StagingPool set the Queue-path staging came from (-1: self-allocated).
    int staging_pool_set() const { return staging_pool_set_; }

    // Timeline trace (off by default; GFD_TRACE=1 or set_trace(true)).
    // Timestamps are CLOCK_MONOTONIC nanoseconds.
    enum TraceKind : uint32_t {
        TRACE_BATCH_FIRST = 1,  // first descriptor of a batch consumed: a = slot, b = read_idx
        TRACE_FLUSH = 2,        // batch handed to the copy path: a = entries, b = bytes
        TRACE_ISSUED = 3,       // batch copies issued: b = fence after them
        TRACE_DONE = 4,         // done_idx published: b = value
        TRACE_GAP_FLUSH = 5,    // partial batch flushed after a gap: a = entries
        TRACE_DIRECT_BEGIN = 6, // submit_direct entered: a = entries, b = bytes
        TRACE_CHUNK = 7,        // a staging chunk's copy issued: a = chunk, b = bytes
        TRACE_DIRECT_END = 8,   // submit_direct returns: b = elapsed ns
        TRACE_GATHER_ENTRY = 9,        // gather job entered
        TRACE_GATHER_IDLE = 10,        // previous job's workers have left
        TRACE_GATHER_PUBLISHED = 11,   // job visible to the workers: a = workers asleep at that moment
        TRACE_GATHER_FIRST_SLICE = 12, // first slice copied: a = threads that copied
        TRACE_GATHER_BUILT = 13,       // job state built (slices cut)
        TRACE_ZC_LAUNCH = 14,          // zero-copy kernel launched or worker job posted: a = entries, b = bytes
        TRACE_ZC_DONE = 15,            // its completion word(s) seen by the host
        TRACE_ZC_CHECKED = 16,         // Queue: a batch's sources and destinations checked for the worker
    };
    struct TraceEvent {
        uint64_t t_ns;
        uint32_t kind;
        uint32_t a;
        uint64_t b;
    };
    void set_trace(bool on);
    // Move up to `max` recorded events (oldest first) into `out`; returns the count.
    int read_trace(TraceEvent* out, int max);

    // SDMA copy timeline: engine start/end of every copy of the Queue path
    // (path 0) and the Direct path (path 1), on copy_clock_ns()'s clock.
    struct CopyTiming {
        uint64_t seq, bytes, start_ns, end_ns;
        uint32_t channel, engine, path, _pad;
    };
    void set_copy_timing(bool on);
    int read_copy_times(CopyTiming* out, int max);
    uint64_t copy_clock_ns() const;
    void trace(uint32_t kind, uint32_t a, uint64_t b);
    void trace_at(uint64_t t_ns, uint32_t kind, uint32_t a, uint64_t b);
    void trace_gather_run();  // the last gather job's phases (when tracing)

    // Host-side effects applied once a batch's copies have completed.
    struct CompletionSlot {
        uint64_t fence = 0;       // every copy below this fence belongs to the batch or earlier
        uint64_t worker_job = 0;  // and every zero-copy worker job up to this one (0: none)
        uint64_t done_value = 0;  // done_idx to publish
        std::vector<std::pair<uint32_t, uint64_t>> host_tiles;  // (tile, progress) for host flags
        std::vector<uint32_t> host_lists;                       // list ids for host flags
        uint32_t lists_done = 0;
        void clear() {
            host_tiles.clear();
            host_lists.clear();
            lists_done = 0;
        }
    };

private:
    struct CompletionFifo;

    void polling_loop();
    void flush_batch(Descriptor* batch, int& batch_count, uint32_t& or_flags);
    bool process_batch(Descriptor* batch, int count);
    void process_batch_tiled(Descriptor* batch, int count, uint64_t cur_read);
    void process_batch_sg(Descriptor* batch, int count, uint64_t cur_read);
    void submit_list(const SGEntry* e, int count, size_t total);
    void submit_list(const SGEntry* e, int count, size_t total, bool dst_contig, bool src_contig, bool uniform);
    // runs == nullptr: destinations contiguous; else nruns destination runs.
    // uniform_hint as for GatherEngine::run.
    bool gather_through_staging(const SGEntry* e, int count, size_t total, const DstRun* runs = nullptr,
                                int nruns = 0, int uniform_hint = -1);
    int direct_scattered(const SGEntry* entries, int count, size_t total, bool uniform);
    int direct_zero_copy(const SGEntry* entries, int count, size_t total, bool uniform, bool sources_checked);
    int direct_worker(const SGEntry* entries, int count, size_t total);
    bool queue_worker_copy(const SGEntry* e, int count, size_t total);
    bool ensure_worker();
    int zc_plan_head(const SGEntry* entries, int count, size_t total, bool uniform, size_t* head_bytes);
    int zc_launch_head(const SGEntry* entries, int k, bool uniform, uint64_t* gen);
    bool zc_sources_pinned(const SGEntry* entries, int count, bool fill_src_table);
    bool ensure_zc_src_table(int count);
    bool zc_dst_in_device(uint64_t lo, uint64_t hi);
    bool zc_ready();
    bool zc_warm_up();
    int zc_wait(uint64_t gen);
    void copy_runs(const SGEntry* e, int count);
    void signal_device_u64(uint64_t* dst, uint64_t value, uint64_t after_begin);
    void publish_done(uint64_t value);
    void push_completion(uint64_t done_value);
    void drain_completions(bool block);
    void finish_slot(CompletionSlot& s);
    bool start_workers();
    bool choose_cpus();

    DescriptorQueue* queue_;
    TiledQueue* tiled_queue_ = nullptr;
    SGTaskQueue* sg_queue_ = nullptr;
    void* gpu_base_;
    void* cpu_base_;
    size_t total_cpu_size_;
    bool use_ce_;
    int numa_node_;
    int core_offset_;
    int num_ce_channels_;
    int exclusive_core_base_;
    int exclusive_core_count_;
    int device_ = 0;

    CopyEngineManager ce_manager_;
    CopyEngineManager direct_ce_manager_;

    // Queue-path staging: rotating buffers; a buffer is reused once the
    // copies out of it (fence) have finished.
    static constexpr int NUM_STAGING_BUFS = 5;
    char* staging_bufs_[NUM_STAGING_BUFS] = {};
    uint64_t staging_fence_[NUM_STAGING_BUFS] = {};
    size_t staging_buffer_size_ = 0;
    int num_staging_bufs_ = 0;
    int staging_cur_ = 0;
    int staging_pool_set_ = -1;
    bool staging_owned_ = false;

    // Direct-path staging (one buffer of total_cpu_size bytes).
    char* direct_staging_ = nullptr;
    size_t direct_staging_size_ = 0;
    size_t direct_chunk_bytes_ = 2u << 20;

    // Pinned source values for flag writes into HBM (ring; a slot is reused
    // only after its copy has finished, which the fence order guarantees once
    // the ring has wrapped past completed fences).
    static constexpr int SIGNAL_SLOTS = 4096;
    uint64_t* signal_values_ = nullptr;
    uint64_t signal_fence_[SIGNAL_SLOTS] = {};
    int signal_next_ = 0;
    // Fence number of the last flag write into HBM: each one is ordered after
    // the previous, so a progress word's final value is its latest.
    uint64_t last_signal_copy_ = CopyEngineManager::kNoFence;
    int list_done_on_device_ = -1;  // -1 unknown, 0 host memory, 1 HBM
    // SG mode: a list whose entries span several batches is "open" from its
    // first batch; its HBM flag waits for every copy since sg_open_begin_.
    bool sg_open_ = false;
    uint64_t sg_open_begin_ = 0;
    int tile_done_on_device_ = -1;

    // Tiled / SG completion bookkeeping.
    uint64_t tile_progress_[MAX_TILES] = {};
    uint64_t tile_marked_[MAX_TILES] = {};

    CompletionFifo* fifo_ = nullptr;
    CompletionSlot pending_;
    std::vector<SGEntry> sg_scratch_;
    std::vector<SGEntry> run_scratch_;
    std::vector<DstRun> queue_runs_;   // destination runs of a Queue-path list
    std::vector<DstRun> direct_runs_;  // destination runs of a Direct-path list
    // Direct path, lists scattered over many destination runs: the entry table
    // in pinned memory for the zero-copy kernel, and its stream.
    SGEntry* zc_table_ = nullptr;
    int zc_table_cap_ = 0;
    gfd_stream_t zc_stream_ = nullptr;
    // Completion of the zero-copy kernels, signalled by the grid's last wave:
    // a wave counter in HBM and the generation word it writes to host memory.
    unsigned int* zc_counter_ = nullptr;
    uint64_t* zc_done_ = nullptr;
    uint64_t zc_gen_ = 0;
    // Small destination-contiguous lists: source addresses (uniform sizes) in
    // pinned memory for the zero-copy tokens kernel.
    uint64_t* zc_src_table_ = nullptr;
    int zc_src_cap_ = 0;
    size_t direct_zc_max_bytes_ = 8u << 20;
    size_t direct_zc_min_bytes_ = 64u << 10;
    size_t direct_zc_head_bytes_ = 2u << 20;
    uint64_t zc_dst_lo_ = 0, zc_dst_hi_ = 0;  // last device allocation found for a destination
    ZcWorker* worker_ = nullptr;
    bool worker_wanted_ = false;  // GFD_ZC_WORKER=1: set up with the copy engines
    size_t worker_queue_max_bytes_ = 4u << 20;
    uint64_t queue_dst_lo_ = 0, queue_dst_hi_ = 0;  // Queue path: last device allocation found
    // The open batch's host and device ranges were looked up when its first
    // descriptor was taken (the flush then keeps them).
    bool batch_checked_ = false;
    uint64_t worker_posted_ = 0;     // Queue path: the last job posted to the worker
    uint64_t worker_done_seen_ = 0;  // and the last one the completion slots saw done
    std::vector<uint32_t> tile_scratch_;
    size_t slice_bytes_ = 0;

    // Gather workers shared by both paths.
    GatherEngine* gather_ = nullptr;
    std::mutex gather_mutex_;
    // Held for a whole submit_direct call: concurrent Direct calls on one
    // poller share the direct staging, run table and zero-copy table, so
    // they run one after the other.
    std::mutex direct_mutex_;
    std::vector<int> worker_cpus_;
    int poller_cpu_ = -1;
    bool cpus_chosen_ = false;

    std::atomic<bool> running_{false};
    std::thread thread_;
    std::function<void()> stop_hook_;

    static constexpr int TRACE_CAP = 16384;
    std::vector<TraceEvent> trace_buf_;
    uint64_t trace_head_ = 0;
    uint64_t trace_tail_ = 0;
    std::atomic<bool> trace_on_{false};
    std::mutex trace_mutex_;

    std::atomic<uint64_t> descriptors_processed_{0};
    std::atomic<uint64_t> batches_submitted_{0};
    std::atomic<uint64_t> coalesced_entries_{0};
    std::atomic<uint64_t> staging_batches_{0};
    std::atomic<uint64_t> total_bytes_copied_{0};
    std::atomic<uint64_t> total_gather_us_{0};
    std::atomic<uint64_t> total_dma_wait_us_{0};
    std::atomic<uint64_t> total_dma_submit_us_{0};
    std::atomic<uint64_t> total_queue_read_us_{0};
};

}  // namespace gfd
