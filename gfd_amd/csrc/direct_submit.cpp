// CpuPollingThread::init_direct_ce / submit_direct: the host-submitted
// ("GFD Direct") path.  Contract as in src/direct_submit.cpp:8-164 of the
// reference: the call blocks until every byte is in HBM and returns the
// elapsed wall time in microseconds (-1 on error).
//
// MI355X design: the destination range is cut into chunks (a short first
// chunk, doubling up to direct_chunk_bytes, 2 MiB by default).  The gather pool fills the pinned
// direct-staging buffer chunk by chunk, every thread working on the oldest
// unfinished chunk, and the calling thread starts the SDMA copy of each
// chunk the moment it is complete, rotating over the copy channels.  Only the
// first chunk's gather and the last chunk's copy are exposed, instead of one
// third of the gather as in the reference's fixed 3-chunk pipeline.
#include <algorithm>
#include <chrono>
#include <cstring>
#include <mutex>

#include "dst_runs.h"
#include "gather_engine.h"
#include "gfd/cpu_polling.h"
#include "gfd/staging_pool.h"
#include "gfd_capi.h"

namespace gfd {

namespace {

struct DirectCtx {
    CpuPollingThread* self;
    CopyEngineManager* ce;
    DevicePtr dst0;
    const char* staging;
    int channels;
    int err;
};

void direct_chunk(void* p, int chunk, size_t off, size_t len) {
    DirectCtx* c = (DirectCtx*)p;
    int e = c->ce->submit_on_channel(chunk % c->channels, c->dst0 + off, c->staging + off, len);
    if (e && !c->err) c->err = e;
    c->self->trace(CpuPollingThread::TRACE_CHUNK, (uint32_t)chunk, len);
}

constexpr size_t kContiguousSplitMin = 8u << 20;  // split one contiguous copy above this

void no_chunk(void*, int, size_t, size_t) {}

}  // namespace

void run_copy_chunk(void* p, int chunk, size_t off, size_t len) {
    RunCopyCtx* c = (RunCopyCtx*)p;
    const size_t end = off + len;
    while (c->cursor < c->nruns) {
        const DstRun& r = c->runs[c->cursor];
        const size_t a = std::max(off, r.off), b = std::min(end, r.off + r.size);
        if (b > a) {
            const int e = c->ce->submit_on_channel(c->next_channel, r.dst + (a - r.off), c->staging + a, b - a);
            c->next_channel = (c->next_channel + 1) % c->channels;
            if (e && !c->err) c->err = e;
        }
        if (r.off + r.size <= end) c->cursor++;
        else break;
    }
    c->self->trace(CpuPollingThread::TRACE_CHUNK, (uint32_t)chunk, len);
}

// Destinations scattered over more runs than are worth one SDMA copy each
// (paged KV caches): the zero-copy kernel writes every entry straight to its
// destination.  Sources that are pinned host memory are read in place;
// otherwise the gather pool first packs them into the (pinned) direct staging
// and the kernel reads from there.  The entry table goes to pinned memory the
// kernel reads.  Returns 0 or an error code.
int CpuPollingThread::direct_scattered(const SGEntry* entries, int count, size_t total, bool uniform) {
    if (zc_table_cap_ < count) {
        if (zc_table_) gfd_hip_host_free(zc_table_);
        zc_table_ = nullptr;
        zc_table_cap_ = 0;
        const int cap = std::max(count, 4096);
        void* t = nullptr;
        if (gfd_hip_host_alloc(&t, (size_t)cap * sizeof(SGEntry), GFD_HOST_DEFAULT) != 0) return -1;
        zc_table_ = static_cast<SGEntry*>(t);
        zc_table_cap_ = cap;
    }
    // Every destination must lie inside one device allocation (the kernel
    // writes them directly); ranges are looked up once per allocation.
    uint64_t dlo = 0, dhi = 0;
    bool pinned = true, any = false;
    for (int i = 0; i < count; i++) {
        if (entries[i].size == 0) continue;
        any = true;
        const uint64_t a = entries[i].dst, b = a + entries[i].size;
        if (a < dlo || b > dhi) {
            uint64_t base = 0, size = 0;
            if (!gfd_hip_device_range(a, &base, &size) || b > base + size) {
                GFD_LOG_ERROR("submit_direct: destination %d is not inside a device allocation\n", i);
                return -1;
            }
            dlo = base;
            dhi = base + size;
        }
        if (pinned && !direct_ce_manager_.host_source_ok(entries[i].src, entries[i].size)) pinned = false;
    }
    if (!any) return 0;  // nothing to move
    if (pinned) {
        std::memcpy(zc_table_, entries, (size_t)count * sizeof(SGEntry));
    } else {
        if (!direct_staging_ || total > direct_staging_size_ || !gather_) return -1;
        {
            std::lock_guard<std::mutex> lock(gather_mutex_);
            gather_->run(entries, count, total, direct_staging_, direct_chunk_bytes_, no_chunk, nullptr,
                         uniform ? 1 : 0);
        }
        size_t off = 0;
        for (int i = 0; i < count; i++) {
            zc_table_[i] = SGEntry{entries[i].dst, direct_staging_ + off, entries[i].size};
            off += entries[i].size;
        }
    }
    if (!zc_stream_ && gfd_hip_stream_create(&zc_stream_) != 0) return -1;
    int rc = gfd_zero_copy_gather(reinterpret_cast<const gfd_sg_entry*>(zc_table_), count, zc_stream_);
    if (rc == 0) rc = gfd_hip_stream_synchronize(zc_stream_);
    return rc;
}

bool CpuPollingThread::init_direct_ce() {
    if (!use_ce_) return false;
    if (gfd_hip_set_device(device_) != 0) return false;
    choose_cpus();
    if (direct_ce_manager_.init(device_, num_ce_channels_) != 0) {
        GFD_LOG_ERROR("direct copy engine init failed\n");
        return false;
    }
    if (!direct_staging_ && total_cpu_size_ > 0) {
        direct_staging_ = StagingPool::alloc_pinned(total_cpu_size_, numa_node_, nullptr);
        if (!direct_staging_) {
            GFD_LOG_ERROR("direct staging allocation of %zu bytes failed\n", total_cpu_size_);
            return false;
        }
        direct_staging_size_ = total_cpu_size_;
    }
    return start_workers();
}

double CpuPollingThread::submit_direct(const SGEntry* entries, int count) {
    if (!direct_ce_manager_.is_initialized() || count <= 0 || !entries) return -1.0;
    std::lock_guard<std::mutex> direct_lock(direct_mutex_);
    const auto t0 = std::chrono::steady_clock::now();
    if (gather_) gather_->prewake();  // workers wake while the list is inspected
    if (direct_ce_manager_.pin_context() != 0) return -1.0;

    // Total bytes and the three list properties the route depends on (split
    // over the gather workers for long lists).
    size_t total = entries[0].size;
    bool dst_contig = true, src_contig = true, uniform = true;
    if (gather_) {
        std::lock_guard<std::mutex> lock(gather_mutex_);
        const GatherEngine::ListScan sc = gather_->scan(entries, count);
        total = sc.total;
        dst_contig = sc.dst_contig;
        src_contig = sc.src_contig;
        uniform = sc.uniform;
    } else {
        for (int i = 1; i < count; i++) {
            const SGEntry& p = entries[i - 1];
            const SGEntry& e = entries[i];
            total += e.size;
            dst_contig &= e.dst == p.dst + p.size;
            src_contig &= (const char*)e.src == (const char*)p.src + p.size;
            uniform &= e.size == p.size;
        }
    }

    // Stamped with the call's entry time (steady_clock is CLOCK_MONOTONIC, the
    // trace clock), so the scan above shows up in the timeline.
    trace_at((uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(t0.time_since_epoch()).count(),
             TRACE_DIRECT_BEGIN, (uint32_t)count, total);
    int err = 0;
    const int nch = direct_ce_manager_.num_channels();
    if (dst_contig && src_contig) {
        // One range: split it over the channels when it is large.
        int parts = total >= kContiguousSplitMin ? nch : 1;
        size_t per = ((total + parts - 1) / parts + 4095) & ~(size_t)4095;
        for (int c = 0; c < parts && !err; c++) {
            size_t off = (size_t)c * per;
            if (off >= total) break;
            size_t len = total - off < per ? total - off : per;
            err = direct_ce_manager_.submit_on_channel(c, entries[0].dst + off,
                                                       (const char*)entries[0].src + off, len);
        }
    } else if (dst_contig && direct_staging_ && total <= direct_staging_size_) {
        std::lock_guard<std::mutex> lock(gather_mutex_);
        if (gather_) {
            DirectCtx ctx{this, &direct_ce_manager_, entries[0].dst, direct_staging_, nch, 0};
            gather_->run(entries, count, total, direct_staging_, direct_chunk_bytes_, direct_chunk, &ctx,
                         uniform ? 1 : 0);
            err = ctx.err;
            trace_gather_run();
        } else {
            size_t off = 0;
            for (int i = 0; i < count; i++) {
                std::memcpy(direct_staging_ + off, entries[i].src, entries[i].size);
                off += entries[i].size;
            }
            err = direct_ce_manager_.submit_on_channel(0, entries[0].dst, direct_staging_, total);
        }
    } else if (!dst_contig && gather_) {
        // Destinations in several runs: a packed gather with one copy per run
        // piece, or the zero-copy kernel when there are many runs.
        const int nr = dst_runs(entries, count, kMaxRunCopies, direct_runs_);
        if (nr <= kMaxRunCopies && direct_staging_ && total <= direct_staging_size_) {
            std::lock_guard<std::mutex> lock(gather_mutex_);
            RunCopyCtx ctx{this, &direct_ce_manager_, direct_staging_, direct_runs_.data(), nr, 0, nch, 0, 0};
            gather_->run(entries, count, total, direct_staging_, direct_chunk_bytes_, run_copy_chunk, &ctx,
                         uniform ? 1 : 0);
            err = ctx.err;
        } else if (nr > kMaxRunCopies) {
            err = direct_scattered(entries, count, total, uniform);
        } else {
            err = direct_ce_manager_.submit_scatter_gather(entries, count);
        }
    } else {
        err = direct_ce_manager_.submit_scatter_gather(entries, count);
    }

    const int werr = direct_ce_manager_.wait_completion();
    const auto t1 = std::chrono::steady_clock::now();
    trace(TRACE_DIRECT_END, 0, (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count());
    if (err || werr) {
        GFD_LOG_ERROR("submit_direct: copy failed (%d / %d)\n", err, werr);
        return -1.0;
    }
    total_bytes_copied_.fetch_add(total, std::memory_order_relaxed);
    descriptors_processed_.fetch_add((uint64_t)count, std::memory_order_relaxed);
    batches_submitted_.fetch_add(1, std::memory_order_relaxed);
    return std::chrono::duration<double, std::micro>(t1 - t0).count();
}

}  // namespace gfd
