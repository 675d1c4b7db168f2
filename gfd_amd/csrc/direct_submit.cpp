// CpuPollingThread::init_direct_ce / submit_direct: the host-submitted
// ("GFD Direct") path.  Contract as in src/direct_submit.cpp:8-164 of the
// reference: the call blocks until every byte is in HBM and returns the
// elapsed wall time in microseconds (-1 on error).
//
// MI355X design: the destination range is cut into chunks
// (direct_chunk_bytes, 2 MiB by default).  The gather pool fills the pinned
// direct-staging buffer chunk by chunk, every thread working on the oldest
// unfinished chunk, and the calling thread starts the SDMA copy of each
// chunk the moment it is complete, rotating over the copy channels.  Only the
// first chunk's gather and the last chunk's copy are exposed, instead of one
// third of the gather as in the reference's fixed 3-chunk pipeline.
#include <chrono>
#include <cstring>
#include <mutex>

#include "gather_engine.h"
#include "gfd/cpu_polling.h"
#include "gfd/staging_pool.h"

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

}  // namespace

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
    const auto t0 = std::chrono::steady_clock::now();
    if (gather_) gather_->prewake();  // workers wake while the list is inspected
    if (direct_ce_manager_.pin_context() != 0) return -1.0;

    size_t total = 0;
    for (int i = 0; i < count; i++) total += entries[i].size;
    bool dst_contig = true, src_contig = true, uniform = true;
    for (int i = 1; i < count; i++) {
        dst_contig &= entries[i].dst == entries[i - 1].dst + entries[i - 1].size;
        src_contig &= (const char*)entries[i].src == (const char*)entries[i - 1].src + entries[i - 1].size;
        uniform &= entries[i].size == entries[0].size;
    }

    trace(TRACE_DIRECT_BEGIN, (uint32_t)count, total);
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
            if (trace_on_.load(std::memory_order_relaxed)) {
                const GatherEngine::RunTimes rt = gather_->last_run();
                trace_at(rt.entry, TRACE_GATHER_ENTRY, 0, 0);
                trace_at(rt.idle, TRACE_GATHER_IDLE, 0, 0);
                trace_at(rt.built, TRACE_GATHER_BUILT, 0, 0);
                trace_at(rt.published, TRACE_GATHER_PUBLISHED, (uint32_t)rt.sleepers, 0);
                trace_at(rt.first_slice, TRACE_GATHER_FIRST_SLICE, (uint32_t)rt.copiers, 0);
            }
        } else {
            size_t off = 0;
            for (int i = 0; i < count; i++) {
                std::memcpy(direct_staging_ + off, entries[i].src, entries[i].size);
                off += entries[i].size;
            }
            err = direct_ce_manager_.submit_on_channel(0, entries[0].dst, direct_staging_, total);
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
