// Host side of WarpSpecSession and SGWarpSpecSession (the reference's
// src/warp_spec_session.cpp:8-142 and src/sg_warp_spec_session.cpp:9-186).
//
// The sessions own their queues (fine-grained host memory, so kernels read
// them with system-scope loads) and HBM arrays (per-tile / per-list
// completion words plus the device counters the kernels claim work from).
// The kernels' transfer waves move the data themselves; the CPU poller a
// session hands out through get_poller() is created on first use and serves
// kernels the caller launches around its start()/stop().
#include <algorithm>
#include <chrono>
#include <cstddef>
#include <cstring>
#include <thread>

#include "gfd/log.h"
#include "gfd/warp_spec_session.h"

namespace gfd {

namespace {

int default_num_blocks() {
    int dev = 0, n = 0;
    gfd_hip_get_device(&dev);
    if (gfd_hip_cu_count(&n, dev) != 0 || n <= 0) n = 1;
    return n;
}

double ms_between(std::chrono::steady_clock::time_point a, std::chrono::steady_clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}

uint64_t load_acquire(const volatile uint64_t* p) { return __atomic_load_n(const_cast<uint64_t*>(p), __ATOMIC_ACQUIRE); }
void store_release(volatile uint64_t* p, uint64_t v) { __atomic_store_n(const_cast<uint64_t*>(p), v, __ATOMIC_RELEASE); }

// Staging of a session's poller: five buffers of this size.  Descriptors of a
// larger batch are copied run by run from their (pinned) sources instead.
constexpr size_t kSessionPollerStaging = 8u << 20;

// A poller over `queue` with its copy engines set up; logs and still returns
// the object if the set-up fails, as the reference's sessions do.
CpuPollingThread* make_session_poller(DescriptorQueue* queue, void* gpu_base, void* cpu_base, size_t staging,
                                      TiledQueue* tiled) {
    auto* p = new CpuPollingThread(queue, gpu_base, cpu_base, staging, true, -1);
    if (tiled) p->set_tiled_queue(tiled);
    if (!p->init_copy_engine()) GFD_LOG_ERROR("session poller: copy engine set-up failed\n");
    return p;
}

}  // namespace

// ============================================================ WarpSpecSession

WarpSpecSession::WarpSpecSession(const WarpSpecConfig& config) : config_(config) {
    // Validation as src/warp_spec_session.cpp:11-23, plus the wave64 block limit.
    if (config_.total_tokens == 0 || config_.token_size == 0) {
        GFD_LOG_ERROR("WarpSpecSession: total_tokens and token_size must be > 0\n");
        return;
    }
    const uint32_t chunk = config_.effective_tokens_per_chunk();
    if (config_.tokens_per_tile == 0 || chunk == 0) {
        GFD_LOG_ERROR("WarpSpecSession: tokens_per_tile and tokens_per_chunk must be > 0\n");
        return;
    }
    if (config_.tokens_per_tile % chunk != 0) {
        GFD_LOG_ERROR("WarpSpecSession: tokens_per_tile must be divisible by tokens_per_chunk\n");
        return;
    }
    if (config_.block_size() > 1024) {
        GFD_LOG_ERROR("WarpSpecSession: %u chunks per tile need %d threads (> 1024)\n", config_.chunks_per_tile(),
                      config_.block_size());
        return;
    }
    if (!config_.cpu_src || !config_.gpu_dst) {
        GFD_LOG_ERROR("WarpSpecSession: cpu_src and gpu_dst are required\n");
        return;
    }
    // Default grid: one workgroup per tile, at most one per CU.  Idle
    // workgroups would only claim nothing and leave.
    num_blocks_ = config_.num_blocks > 0
                      ? config_.num_blocks
                      : std::max(1, std::min(default_num_blocks(), (int)std::max<uint32_t>(1, config_.total_tiles())));
    if (config_.transfer_helper_waves < 0)
        config_.transfer_helper_waves =
            auto_helper_waves(std::min(num_blocks_, (int)std::max<uint32_t>(1, config_.total_tiles())));

    void* q = nullptr;
    if (gfd_hip_host_alloc(&q, sizeof(TiledQueue), GFD_HOST_COHERENT) != 0) {
        GFD_LOG_ERROR("WarpSpecSession: TiledQueue allocation failed\n");
        return;
    }
    tq_ = static_cast<TiledQueue*>(q);
    std::memset((void*)tq_, 0, sizeof(TiledQueue));
    tq_->scheduler.total_tiles = config_.total_tiles();
    tq_->scheduler.tokens_per_tile = config_.tokens_per_tile;
    tq_->scheduler.tokens_per_chunk = chunk;
    tq_->scheduler.chunks_per_tile = config_.chunks_per_tile();
    tq_->scheduler.token_size = config_.token_size;

    const size_t words = (size_t)MAX_TILES + TILE_DEVICE_COUNTER_WORDS;
    void* d = nullptr;
    if (gfd_hip_malloc(&d, words * sizeof(uint64_t)) != 0) {
        GFD_LOG_ERROR("WarpSpecSession: device signal allocation failed\n");
        return;
    }
    d_signals_ = static_cast<uint64_t*>(d);
    gfd_hip_memset_d8((uint64_t)(uintptr_t)d_signals_, 0, words * sizeof(uint64_t));
    tq_->d_tile_chunk_done = d_signals_;
    ok_ = true;
}

WarpSpecSession::~WarpSpecSession() {
    if (running_) synchronize();
    delete poller_;
    poller_ = nullptr;
    if (d_signals_) gfd_hip_free(d_signals_);
    if (tq_) gfd_hip_host_free(tq_);
}

WarpSpecSession::LaunchParams WarpSpecSession::get_launch_params() const {
    LaunchParams p;
    p.tq = tq_;
    p.gpu_buffer = config_.gpu_dst;
    p.cpu_base = config_.cpu_src;
    p.grid = (unsigned)num_blocks_;
    p.block = (unsigned)config_.block_size();
    return p;
}

void WarpSpecSession::reset() {
    if (running_) synchronize();
    if (!tq_) return;
    if (d_signals_)
        gfd_hip_memset_d8((uint64_t)(uintptr_t)d_signals_, 0,
                          ((size_t)MAX_TILES + TILE_DEVICE_COUNTER_WORDS) * sizeof(uint64_t));
    std::memset((void*)tq_->tile_chunk_done, 0, sizeof(tq_->tile_chunk_done));
    tq_->scheduler.next_tile = 0;
    error_bits_ = 0;
    tiles_done_ = 0;
    landed_tiles_total_ = 0;
    if (poller_) poller_->reset_stats();
}

CpuPollingThread* WarpSpecSession::get_poller() const {
    if (!poller_ && ok_) {
        const size_t total = (size_t)config_.total_tokens * config_.token_size;
        poller_ = make_session_poller(&tq_->base, config_.gpu_dst, config_.cpu_src,
                                      std::min(total, kSessionPollerStaging), tq_);
        const uint64_t tokens = landed_tiles_total_ * config_.tokens_per_tile;
        poller_->add_device_landed(tokens, tokens * config_.token_size, landed_tiles_total_);
    }
    return poller_;
}

void WarpSpecSession::before_launch(gfd_stream_t stream) {
    reset();  // as the reference's launch (warp_spec_session.h:217)
    stream_ = stream;
    launch_time_ = std::chrono::steady_clock::now();
    running_ = ok_;
}

bool WarpSpecSession::synchronize() {
    if (!running_) return ok_ && error_bits_ == 0 && tiles_done_ == config_.total_tiles();
    const int rc = gfd_hip_stream_synchronize(stream_);
    last_elapsed_ms_ = ms_between(launch_time_, std::chrono::steady_clock::now());
    running_ = false;
    TileDeviceCounters c{};
    if (rc == 0 && gfd_hip_memcpy_d2h(&c, (uint64_t)(uintptr_t)(d_signals_ + MAX_TILES), sizeof(c)) == 0) {
        error_bits_ = c.error;
        tiles_done_ = c.tiles_done;
        // Host-visible progress mirror (tile_chunk_done, tiled_queue.h:41).
        const uint32_t n = std::min<uint32_t>(config_.total_tiles(), (uint32_t)MAX_TILES);
        if (n) gfd_hip_memcpy_d2h((void*)tq_->tile_chunk_done, (uint64_t)(uintptr_t)d_signals_, n * sizeof(uint64_t));
        tq_->scheduler.next_tile = (uint32_t)std::min<uint64_t>(c.next_tile, config_.total_tiles());
        landed_tiles_total_ += tiles_done_;
        if (poller_) {
            const uint64_t tokens = tiles_done_ * config_.tokens_per_tile;
            poller_->add_device_landed(tokens, tokens * config_.token_size, tiles_done_);
        }
    } else {
        GFD_LOG_ERROR("WarpSpecSession: synchronize failed: %s\n", gfd_hip_error_string(rc));
        error_bits_ |= 1ull << 63;
    }
    if (error_bits_) GFD_LOG_ERROR("WarpSpecSession: kernel reported error bits 0x%llx\n", (unsigned long long)error_bits_);
    return error_bits_ == 0 && tiles_done_ == config_.total_tiles();
}

WarpSpecSession::Stats WarpSpecSession::get_stats() const {
    Stats s;
    s.descriptors_processed = tiles_done_ * config_.tokens_per_tile;
    s.bytes_transferred = s.descriptors_processed * (uint64_t)config_.token_size;
    s.elapsed_ms = running_ ? ms_between(launch_time_, std::chrono::steady_clock::now()) : last_elapsed_ms_;
    s.bandwidth_gbps = s.elapsed_ms > 0 ? (double)s.bytes_transferred / (s.elapsed_ms * 1e6) : 0.0;
    return s;
}

// ========================================================== SGWarpSpecSession

SGWarpSpecSession::SGWarpSpecSession(const SGWarpSpecConfig& config) : config_(config) {
    if (config_.transfer_helper_waves > 3) {  // SG_MAX_HELPERS
        GFD_LOG_ERROR("SGWarpSpecSession: transfer_helper_waves must be 0..3 (got %d)\n", config_.transfer_helper_waves);
        return;
    }
    if (config_.block_size() > 512) {  // SG_MAX_BLOCK of sg_warp_spec.h
        GFD_LOG_ERROR("SGWarpSpecSession: %d compute + %d helper waves exceed a 512-thread workgroup\n",
                      config_.num_compute_warps, config_.transfer_helper_waves);
        return;
    }
    // Default grid: 64 workgroups (8 per XCD).  64 transfer waves with 16
    // loads in flight each keep the PCIe link full; more only add idle
    // pollers (measured: 55 GB/s at 32-64 workgroups, 47-53 at 256).
    num_blocks_ = config_.num_blocks > 0 ? config_.num_blocks : std::min(default_num_blocks(), 64);
    if (config_.transfer_helper_waves < 0) config_.transfer_helper_waves = auto_helper_waves(num_blocks_);
    void* q = nullptr;
    if (gfd_hip_host_alloc(&q, sizeof(SGTaskQueue), GFD_HOST_COHERENT) != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: SGTaskQueue allocation failed\n");
        return;
    }
    sq_ = static_cast<SGTaskQueue*>(q);
    std::memset((void*)sq_, 0, sizeof(SGTaskQueue));
    sq_->idle_limit_ms = config_.idle_limit_ms;
    if (gfd_hip_host_alloc(&q, sizeof(DescriptorQueue), GFD_HOST_COHERENT) != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: DescriptorQueue allocation failed\n");
        return;
    }
    dq_ = static_cast<DescriptorQueue*>(q);
    std::memset((void*)dq_, 0, sizeof(DescriptorQueue));
    const size_t words = (size_t)MAX_SG_LISTS + SG_DEVICE_COUNTER_WORDS;
    void* d = nullptr;
    if (gfd_hip_malloc(&d, words * sizeof(uint64_t)) != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: d_list_done allocation failed\n");
        return;
    }
    sq_->d_list_done = static_cast<uint64_t*>(d);
    gfd_hip_memset_d8((uint64_t)(uintptr_t)d, 0, words * sizeof(uint64_t));
    ok_ = true;
}

SGWarpSpecSession::~SGWarpSpecSession() {
    if (running_) synchronize();
    delete poller_;  // clears its stop hook first
    poller_ = nullptr;
    if (trace_buf_) gfd_hip_free(trace_buf_);
    if (dev_ring_) gfd_hip_free(dev_ring_);
    if (sq_) {
        if (sq_->d_list_done) gfd_hip_free(sq_->d_list_done);
        gfd_hip_host_free(sq_);
    }
    if (dq_) gfd_hip_host_free(dq_);
}

SGTaskQueue* SGWarpSpecSession::device_ring() {
    if (dev_ring_ || !ok_) return dev_ring_;
    void* d = nullptr;
    if (gfd_hip_malloc(&d, sizeof(SGTaskQueue)) != 0) return nullptr;
    // Zeroed (no list committed in any slot), sharing the host queue's
    // d_list_done and device counters.
    uint64_t* done = sq_->d_list_done;
    if (gfd_hip_memset_d8((uint64_t)(uintptr_t)d, 0, sizeof(SGTaskQueue)) != 0 ||
        gfd_hip_memcpy_h2d((uint64_t)(uintptr_t)d + offsetof(SGTaskQueue, d_list_done), &done, sizeof(done)) != 0) {
        gfd_hip_free(d);
        return nullptr;
    }
    dev_ring_ = static_cast<SGTaskQueue*>(d);
    return dev_ring_;
}

bool SGWarpSpecSession::list_done(uint64_t idx) const {
    return load_acquire(&sq_->lists[idx % MAX_SG_LISTS].done) >= idx + 1;
}

void SGWarpSpecSession::retire_done() {
    while (!pending_.empty() && list_done(pending_.front().idx)) pending_.pop_front();
}

bool SGWarpSpecSession::wait_until(const std::function<bool()>& cond, double limit_ms) {
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t n = 0;; n++) {
        if (cond()) return true;
        if (n > 256) {
            if (ms_between(t0, std::chrono::steady_clock::now()) > limit_ms) return false;
            std::this_thread::sleep_for(std::chrono::microseconds(20));
        }
    }
}

double SGWarpSpecSession::wait_limit_ms() const {
    return (config_.idle_limit_ms ? (double)config_.idle_limit_ms : 30000.0) + 10000.0;
}

uint64_t SGWarpSpecSession::submit_sg_list(const DeviceSGEntry* entries, uint32_t count, uint32_t list_id,
                                           uint32_t flags) {
    // src/sg_warp_spec_session.cpp:81-116, with backpressure: the ring slot's
    // previous list and the pool entries being reused must have landed.
    if (!ok_ || (count > 0 && !entries) || count > (uint32_t)MAX_SG_POOL_ENTRIES) {
        GFD_LOG_ERROR("SGWarpSpecSession::submit_sg_list: invalid argument\n");
        return ~0ull;
    }
    const uint64_t idx = sq_->list_alloc_idx;
    const uint64_t pool = sq_->entry_alloc_idx;
    retire_done();
    auto room = [&]() {
        retire_done();
        if (idx >= (uint64_t)MAX_SG_LISTS && !list_done(idx - MAX_SG_LISTS)) return false;
        return pending_.empty() || pool + count - pending_.front().pool_begin <= (uint64_t)MAX_SG_POOL_ENTRIES;
    };
    if (!room()) {
        if (!running_) {
            GFD_LOG_ERROR("SGWarpSpecSession::submit_sg_list: ring or pool full and no kernel running\n");
            return ~0ull;
        }
        if (!wait_until(room, wait_limit_ms())) {
            GFD_LOG_ERROR("SGWarpSpecSession::submit_sg_list: timed out waiting for ring / pool space\n");
            return ~0ull;
        }
    }
    for (uint32_t i = 0; i < count; i++) sq_->entries[(pool + i) % MAX_SG_POOL_ENTRIES] = entries[i];
    SGList& l = sq_->lists[idx % MAX_SG_LISTS];
    l.pool_offset = (uint32_t)(pool % MAX_SG_POOL_ENTRIES);
    l.count = count;
    l.list_id = list_id;
    l.flags = flags;
    store_release(&l.sequence, idx + 1);  // commit
    sq_->entry_alloc_idx = pool + count;
    sq_->list_alloc_idx = idx + 1;
    pending_.push_back(Pending{idx, pool, count});
    return idx;
}

void SGWarpSpecSession::before_launch(gfd_stream_t stream, int helper_waves, int compute_waves, uint32_t deadline_ms,
                                      SGTaskQueue* gpu_ring) {
    if (running_) synchronize();
    if (!ok_) return;
    __atomic_store_n(&sq_->terminate, 0u, __ATOMIC_RELEASE);
    sq_->lists_completed = 0;
    dq_->write_idx = dq_->read_idx = dq_->done_idx = 0;
    // Device counters: claims start at the first list no launch has consumed;
    // GPU submitters allocate after the lists the host has already queued.
    SGDeviceCounters c{};
    c.list_claim = consumed_lists_;
    c.list_alloc = sq_->list_alloc_idx;
    c.entry_alloc = c.entry_first = sq_->entry_alloc_idx;
    c.entries_done = consumed_entries_;
    c.list_known = consumed_lists_;
    c.list_base = consumed_lists_;
    c.helpers = (uint64_t)(helper_waves < 0 ? config_.transfer_helper_waves : helper_waves);
    c.compute_waves = (uint64_t)(compute_waves < 0 ? this->compute_waves() : compute_waves);
    c.host_lists = sq_->list_alloc_idx - consumed_lists_;
    c.idle_ticks = sg_idle_ticks(sq_->idle_limit_ms);
    // Relative here (100 MHz ticks); the set-up kernel adds the GPU clock.
    c.deadline = (uint64_t)deadline_ms * 100000ull;
    c.dev_ring = gpu_ring && gpu_ring == dev_ring_ ? (uint64_t)(uintptr_t)gpu_ring : 0;
    uint64_t trace_words = 0;
    if (trace_buf_) {
        c.trace = (uint64_t)(uintptr_t)trace_buf_;
        c.trace_cap = trace_cap_;
        c.trace_blocks = (uint64_t)num_blocks_;
        trace_words = ((uint64_t)trace_cap_ * sizeof(SGTraceList) + (uint64_t)num_blocks_ * sizeof(SGTraceBlock)) / 8;
    }
    // On the launch stream, ahead of the kernel: no host wait per launch.
    // Should that launch fail, the same state is written with blocking
    // copies instead, so the kernel never starts on stale counters.
    int rc = gfd_sg_prepare_launch(sq_->d_list_done, &c, static_cast<uint64_t*>(trace_buf_), trace_words, stream);
    if (rc != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: launch set-up kernel failed (%s); writing the state directly\n",
                      gfd_hip_error_string(rc));
        rc = gfd_hip_stream_synchronize(stream);
        c.deadline = 0;  // the host cannot read the GPU clock: no launch deadline this time
        if (!rc && trace_words) rc = gfd_hip_memset_d8(c.trace, 0, trace_words * 8);
        if (!rc) rc = gfd_hip_memset_d8((uint64_t)(uintptr_t)sq_->d_list_done, 0, MAX_SG_LISTS * sizeof(uint64_t));
        if (!rc) rc = gfd_hip_memcpy_h2d((uint64_t)(uintptr_t)sg_device_counters(sq_), &c, sizeof(c));
        if (!rc) rc = gfd_hip_device_synchronize();
        if (rc) {
            GFD_LOG_ERROR("SGWarpSpecSession: launch set-up failed: %s\n", gfd_hip_error_string(rc));
            error_bits_ |= 1ull << 63;
        }
    }
    stream_ = stream;
    launch_time_ = std::chrono::steady_clock::now();
    running_ = true;
}

bool SGWarpSpecSession::synchronize(uint64_t extra_gpu_lists) {
    if (!running_) return ok_ && error_bits_ == 0;
    // As src/sg_warp_spec_session.cpp:118-139: every submitted list lands,
    // then terminate releases the transfer waves.
    const uint64_t host_end = sq_->list_alloc_idx;
    bool landed = wait_until(
        [&]() {
            retire_done();
            if (!pending_.empty()) return false;
            for (uint64_t i = 0; i < extra_gpu_lists; i++)
                if (!list_done(host_end + i)) return false;
            return true;
        },
        wait_limit_ms());
    __atomic_store_n(&sq_->terminate, 1u, __ATOMIC_RELEASE);
    const int rc = gfd_hip_stream_synchronize(stream_);
    last_elapsed_ms_ = ms_between(launch_time_, std::chrono::steady_clock::now());
    running_ = false;
    SGDeviceCounters c{};
    if (rc != 0 || gfd_hip_memcpy_d2h(&c, (uint64_t)(uintptr_t)sg_device_counters(sq_), sizeof(c)) != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: synchronize failed: %s\n", gfd_hip_error_string(rc));
        error_bits_ |= 1ull << 63;
        return false;
    }
    absorb(c);
    // A kernel the caller launches next, without launch(), starts from here.
    if (poller_) prepare_raw_launch();
    if (!landed || !pending_.empty()) {
        GFD_LOG_ERROR("SGWarpSpecSession: %zu submitted lists did not land\n", pending_.size());
        pending_.clear();
        landed = false;
    }
    if (error_bits_) GFD_LOG_ERROR("SGWarpSpecSession: kernel reported error bits 0x%llx\n", (unsigned long long)error_bits_);
    return landed && error_bits_ == 0;
}

void SGWarpSpecSession::absorb(const SGDeviceCounters& c) {
    error_bits_ |= c.error;
    entries_done_ = c.entries_done - consumed_entries_;
    bytes_done_ = c.bytes_done;
    lists_done_ = c.lists_done;
    // Everything committed so far has been consumed (unless a wait gave up).
    consumed_lists_ = std::max<uint64_t>((uint64_t)sq_->list_alloc_idx, c.list_alloc);
    consumed_entries_ = std::max<uint64_t>((uint64_t)sq_->entry_alloc_idx, c.entry_alloc);
    sq_->list_alloc_idx = consumed_lists_;
    sq_->entry_alloc_idx = consumed_entries_;
    sq_->list_read_idx = consumed_lists_;
    sq_->entry_consumed_idx = consumed_entries_;
    sq_->lists_completed = lists_done_;
    retire_done();
    landed_entries_total_ += entries_done_;
    landed_bytes_total_ += bytes_done_;
    landed_lists_total_ += lists_done_;
    if (poller_) poller_->add_device_landed(entries_done_, bytes_done_, lists_done_);
}

void SGWarpSpecSession::prepare_raw_launch() {
    __atomic_store_n(&sq_->terminate, 0u, __ATOMIC_RELEASE);
    SGDeviceCounters c{};
    c.list_claim = c.list_known = c.list_base = consumed_lists_;
    c.list_alloc = sq_->list_alloc_idx;
    c.entry_alloc = c.entry_first = sq_->entry_alloc_idx;
    c.entries_done = consumed_entries_;
    c.compute_waves = 1;  // the caller's kernel layout is its own: no helpers, one compute wave
    c.host_lists = sq_->list_alloc_idx - consumed_lists_;
    c.idle_ticks = sg_idle_ticks(sq_->idle_limit_ms);
    const uint64_t d = (uint64_t)(uintptr_t)sq_->d_list_done;
    if (gfd_hip_memset_d8(d, 0, MAX_SG_LISTS * sizeof(uint64_t)) != 0 ||
        gfd_hip_memcpy_h2d((uint64_t)(uintptr_t)sg_device_counters(sq_), &c, sizeof(c)) != 0 ||
        gfd_hip_device_synchronize() != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: writing the counters for the next launch failed\n");
        error_bits_ |= 1ull << 63;
    }
}

void SGWarpSpecSession::after_raw_launch() {
    // A launch made through launch() is taken in by synchronize().
    if (!ok_ || running_) return;
    SGDeviceCounters c{};
    if (gfd_hip_memcpy_d2h(&c, (uint64_t)(uintptr_t)sg_device_counters(sq_), sizeof(c)) != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: reading the device counters failed\n");
        error_bits_ |= 1ull << 63;
        return;
    }
    // Every transfer wave claims at least one ring index before it can see
    // terminate, so an untouched claim counter means no kernel ran.
    if (c.list_claim == c.list_base && c.lists_done == 0 && c.error == 0) return;
    absorb(c);
    if (error_bits_) GFD_LOG_ERROR("SGWarpSpecSession: kernel reported error bits 0x%llx\n", (unsigned long long)error_bits_);
    prepare_raw_launch();
}

CpuPollingThread* SGWarpSpecSession::get_poller() const {
    if (!poller_ && ok_) {
        auto* self = const_cast<SGWarpSpecSession*>(this);
        poller_ = make_session_poller(dq_, nullptr, nullptr, kSessionPollerStaging, nullptr);
        poller_->add_device_landed(landed_entries_total_, landed_bytes_total_, landed_lists_total_);
        poller_->set_stop_hook([self]() { self->after_raw_launch(); });
    }
    return poller_;
}

void SGWarpSpecSession::reset() {
    if (running_) synchronize();
    if (!sq_) return;
    uint64_t* d = sq_->d_list_done;
    const uint32_t idle = sq_->idle_limit_ms;
    std::memset((void*)sq_, 0, sizeof(SGTaskQueue));
    sq_->d_list_done = d;
    sq_->idle_limit_ms = idle;
    if (dq_) std::memset((void*)dq_, 0, sizeof(DescriptorQueue));
    // Waited for: the next launch's set-up runs on the caller's stream, which
    // need not be ordered after the null stream this memset runs on.
    if (d) {
        gfd_hip_memset_d8((uint64_t)(uintptr_t)d, 0, ((size_t)MAX_SG_LISTS + SG_DEVICE_COUNTER_WORDS) * sizeof(uint64_t));
        gfd_hip_stream_synchronize(nullptr);
    }
    pending_.clear();
    consumed_lists_ = consumed_entries_ = 0;
    error_bits_ = entries_done_ = bytes_done_ = lists_done_ = 0;
    landed_entries_total_ = landed_bytes_total_ = landed_lists_total_ = 0;
    if (poller_) poller_->reset_stats();
}

bool SGWarpSpecSession::gpu_lists_fit(uint64_t lists, uint64_t entries) const {
    const uint64_t host_lists = sq_ ? sq_->list_alloc_idx - consumed_lists_ : 0;
    const uint64_t host_entries = sq_ ? sq_->entry_alloc_idx - consumed_entries_ : 0;
    return host_lists + lists < (uint64_t)MAX_SG_LISTS - 1 && host_entries + entries <= (uint64_t)MAX_SG_POOL_ENTRIES;
}

bool SGWarpSpecSession::enable_trace(uint32_t max_lists) {
    if (running_) synchronize();
    if (trace_buf_) gfd_hip_free(trace_buf_);
    trace_buf_ = nullptr;
    trace_cap_ = 0;
    if (!ok_ || max_lists == 0) return ok_;
    void* d = nullptr;
    const size_t bytes = (size_t)max_lists * sizeof(SGTraceList) + (size_t)num_blocks_ * sizeof(SGTraceBlock);
    if (gfd_hip_malloc(&d, bytes) != 0) {
        GFD_LOG_ERROR("SGWarpSpecSession: trace buffer allocation failed\n");
        return false;
    }
    gfd_hip_memset_d8((uint64_t)(uintptr_t)d, 0, bytes);
    gfd_hip_stream_synchronize(nullptr);
    trace_buf_ = d;
    trace_cap_ = max_lists;
    return true;
}

bool SGWarpSpecSession::read_trace(std::vector<SGTraceList>& lists, std::vector<SGTraceBlock>& blocks) const {
    lists.clear();
    blocks.clear();
    if (!trace_buf_ || running_) return false;
    lists.resize(trace_cap_);
    blocks.resize((size_t)num_blocks_);
    const uint64_t base = (uint64_t)(uintptr_t)trace_buf_;
    if (gfd_hip_memcpy_d2h(lists.data(), base, lists.size() * sizeof(SGTraceList)) != 0 ||
        gfd_hip_memcpy_d2h(blocks.data(), base + lists.size() * sizeof(SGTraceList),
                           blocks.size() * sizeof(SGTraceBlock)) != 0) {
        lists.clear();
        blocks.clear();
        return false;
    }
    return true;
}

SGWarpSpecSession::Stats SGWarpSpecSession::get_stats() const {
    Stats s;
    s.descriptors_processed = entries_done_;
    s.bytes_transferred = bytes_done_;
    s.elapsed_ms = running_ ? ms_between(launch_time_, std::chrono::steady_clock::now()) : last_elapsed_ms_;
    s.bandwidth_gbps = s.elapsed_ms > 0 ? (double)s.bytes_transferred / (s.elapsed_ms * 1e6) : 0.0;
    return s;
}

}  // namespace gfd
