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
#include <climits>
#include <cstdlib>
#include <immintrin.h>
#include <cstring>
#include <mutex>

#include "dst_runs.h"
#include "gather_engine.h"
#include "gfd/cpu_polling.h"
#include "gfd/staging_pool.h"
#include "gfd_capi.h"
#include "zc_worker.h"

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
constexpr int kZcNotTaken = INT_MIN;               // direct_zero_copy: the list does not qualify

}  // namespace

// The zero-copy SG kernel (and the zero-copy worker) gives each entry of a
// short list a wave of its own, so a list of fewer entries than its `waves`
// waves leaves waves idle while a few stream whole large entries.  Such a
// list's entries are cut into pieces of at least 4 KiB, a multiple of 16
// bytes each (an entry's last piece takes what is left), so the pieces keep
// each entry's alignment.  The piece size is set for waves - count waves,
// since each entry's last piece may be a short one: the table then has at
// most `waves` records, one per wave (*presliced = true; the kernel's
// presliced launch does not cut them again).  Writes the table to out (at
// most cap records) and returns its length, or copies the entries unchanged
// (*presliced = false) when the list is long enough or the pieces would not
// fit.  The caller guarantees count <= cap.
int zc_fill_sg_table(const SGEntry* in, int count, size_t total, SGEntry* out, int cap, bool* presliced, int waves) {
    constexpr size_t kMinPiece = 4096;
    *presliced = false;
    if (count < waves && total / (size_t)count >= 2 * kMinPiece) {
        const size_t free_waves = (size_t)(waves - count);
        const size_t piece = std::max(kMinPiece, ((total + free_waves - 1) / free_waves + 15) & ~(size_t)15);
        int n = 0;
        for (int i = 0; i < count && n >= 0; i++) {
            for (size_t off = 0; off < in[i].size; off += piece) {
                if (n == cap) {
                    n = -1;
                    break;
                }
                const size_t len = std::min(piece, in[i].size - off);
                out[n++] = SGEntry{in[i].dst + off, (const char*)in[i].src + off, len};
            }
        }
        if (n >= 0) {
            *presliced = true;
            return n;
        }
    }
    std::memcpy(out, in, (size_t)count * sizeof(SGEntry));
    return count;
}

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

// Zero-copy completion state: the HBM wave counter and the host word the
// grid's last wave raises (allocated once per poller).
bool CpuPollingThread::zc_ready() {
    if (zc_done_ && zc_counter_ && zc_stream_) return true;
    if (!zc_stream_ && gfd_hip_stream_create(&zc_stream_) != 0) return false;
    if (!zc_done_) {
        void* h = nullptr;
        if (gfd_hip_host_alloc(&h, 64, GFD_HOST_COHERENT) != 0) return false;
        std::memset(h, 0, 64);
        zc_done_ = static_cast<uint64_t*>(h);
    }
    if (!zc_counter_) {
        void* d = nullptr;
        if (gfd_hip_malloc(&d, 256) != 0) return false;
        if (gfd_hip_memset_d8((uint64_t)(uintptr_t)d, 0, 256) != 0 || gfd_hip_device_synchronize() != 0) {
            gfd_hip_free(d);
            return false;
        }
        zc_counter_ = static_cast<unsigned int*>(d);
    }
    return true;
}

// Everything the zero-copy route sets up on its first use, done ahead of it:
// the stream and completion words, both address tables, and one 16-byte
// launch of each kernel the route uses (the first launch of a kernel loads
// its code object and creates the stream's hardware queue, ~0.5 ms).  The
// launches copy 16 unused bytes of the pinned completion page into the unused
// upper half of the 256-byte counter allocation.
bool CpuPollingThread::zc_warm_up() {
    if (!zc_ready() || !ensure_zc_src_table(4096)) return false;
    if (zc_table_cap_ < 4096) {
        if (zc_table_) gfd_hip_host_free(zc_table_);
        zc_table_ = nullptr;
        zc_table_cap_ = 0;
        void* t = nullptr;
        if (gfd_hip_host_alloc(&t, 4096 * sizeof(SGEntry), GFD_HOST_DEFAULT) != 0) return false;
        zc_table_ = static_cast<SGEntry*>(t);
        zc_table_cap_ = 4096;
    }
    char* spare_src = reinterpret_cast<char*>(zc_done_) + 32;
    const uint64_t spare_dst = (uint64_t)(uintptr_t)zc_counter_ + 128;
    zc_src_table_[0] = (uint64_t)(uintptr_t)spare_src;
    uint64_t gen = ++zc_gen_;
    if (gfd_zero_copy_gather_tokens_signal(zc_src_table_, (void*)(uintptr_t)spare_dst, 16, 1, zc_counter_, zc_done_,
                                           gen, zc_stream_) != 0 ||
        zc_wait(gen) != 0)
        return false;
    zc_table_[0] = SGEntry{spare_dst + 16, spare_src, 16};
    gen = ++zc_gen_;
    return gfd_zero_copy_gather_signal(reinterpret_cast<const gfd_sg_entry*>(zc_table_), 1, zc_counter_, zc_done_,
                                       gen, zc_stream_) == 0 &&
           zc_wait(gen) == 0;
}

// Wait until the grid launched with generation `gen` has raised the host
// word (every byte it wrote is then in HBM).  Bounded: after
// GFD_DIRECT_TIMEOUT_MS (10 s) the stream is synchronised to surface the
// error and -1 (or the stream's error) is returned.
int CpuPollingThread::zc_wait(uint64_t gen) {
    static const uint64_t limit_us = [] {
        const char* v = std::getenv("GFD_DIRECT_TIMEOUT_MS");
        return (uint64_t)std::max(1ll, v && *v ? std::atoll(v) : 10000ll) * 1000ull;
    }();
    const auto t0 = std::chrono::steady_clock::now();
    for (unsigned i = 1;; i++) {
        if (__atomic_load_n(zc_done_, __ATOMIC_ACQUIRE) == gen) return 0;
        _mm_pause();
        if ((i & 4095) == 0 &&
            (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0)
                    .count() > limit_us) {
            const int rc = gfd_hip_stream_synchronize(zc_stream_);
            if (__atomic_load_n(zc_done_, __ATOMIC_ACQUIRE) == gen) return rc;
            GFD_LOG_ERROR("zero-copy gather did not signal completion (stream status %d)\n", rc);
            return rc ? rc : -1;
        }
    }
}

// Every source lies in pinned host memory the GPU reads at its host address.
// Checked against the last pinned range found, entry by entry; with
// fill_src_table the sources are also written to zc_src_table_ (uniform lists).
// zc_src_table_ holds at least `count` addresses (pinned memory the kernel reads).
bool CpuPollingThread::ensure_zc_src_table(int count) {
    if (zc_src_cap_ >= count) return true;
    if (zc_src_table_) gfd_hip_host_free(zc_src_table_);
    zc_src_table_ = nullptr;
    zc_src_cap_ = 0;
    const int cap = std::max(count, 4096);
    void* t = nullptr;
    if (gfd_hip_host_alloc(&t, (size_t)cap * sizeof(uint64_t), GFD_HOST_DEFAULT) != 0) return false;
    zc_src_table_ = static_cast<uint64_t*>(t);
    zc_src_cap_ = cap;
    return true;
}

bool CpuPollingThread::zc_sources_pinned(const SGEntry* entries, int count, bool fill_src_table) {
    if (fill_src_table && !ensure_zc_src_table(count)) return false;
    uintptr_t lo = 1, hi = 0;  // empty range: the first entry looks it up
    for (int i = 0; i < count; i++) {
        const uintptr_t a = (uintptr_t)entries[i].src, b = a + entries[i].size;
        if (a < lo || b > hi) {
            if (!direct_ce_manager_.host_source_ok(entries[i].src, entries[i].size)) return false;
            direct_ce_manager_.last_pinned_range(&lo, &hi);
            if (a < lo || b > hi) lo = a, hi = b;
        }
        if (fill_src_table) zc_src_table_[i] = (uint64_t)a;
    }
    return true;
}

// [lo, hi) lies inside one device allocation.
bool CpuPollingThread::zc_dst_in_device(uint64_t lo, uint64_t hi) {
    if (lo >= zc_dst_lo_ && hi <= zc_dst_hi_) return true;
    uint64_t base = 0, size = 0;
    if (!gfd_hip_device_range(lo, &base, &size) || hi > base + size) return false;
    zc_dst_lo_ = base;
    zc_dst_hi_ = base + size;
    return true;
}

// Small destination-contiguous list with pinned sources: the zero-copy
// kernel reads the tokens over PCIe and writes them to HBM; its last wave
// raises zc_done_.  Uniform lists pass only their source addresses (8 bytes
// per token); others pass the whole entry table.  Returns 0, kZcNotTaken
// when the list does not qualify (the caller then takes the staged route), or
// an error.
int CpuPollingThread::direct_zero_copy(const SGEntry* entries, int count, size_t total, bool uniform,
                                       bool sources_checked) {
    if (!zc_ready()) return kZcNotTaken;
    if (!zc_dst_in_device(entries[0].dst, entries[0].dst + total)) return kZcNotTaken;
    if (!sources_checked && !zc_sources_pinned(entries, count, uniform)) return kZcNotTaken;
    const uint64_t gen = ++zc_gen_;
    int rc;
    if (uniform) {
        rc = gfd_zero_copy_gather_tokens_signal(zc_src_table_, (void*)(uintptr_t)entries[0].dst,
                                                (uint32_t)entries[0].size, count, zc_counter_, zc_done_, gen,
                                                zc_stream_);
    } else {
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
        bool cut = false;
        static const int kWaves = gfd_zero_copy_target_waves();
        const int n = zc_fill_sg_table(entries, count, total, zc_table_, zc_table_cap_, &cut, kWaves);
        rc = (cut ? gfd_zero_copy_gather_signal_presliced : gfd_zero_copy_gather_signal)(
            reinterpret_cast<const gfd_sg_entry*>(zc_table_), n, zc_counter_, zc_done_, gen, zc_stream_);
    }
    if (rc != 0) return rc;
    trace(TRACE_ZC_LAUNCH, (uint32_t)count, total);
    rc = zc_wait(gen);
    trace(TRACE_ZC_DONE, 0, gen);
    return rc;
}

// The persistent zero-copy worker copies a destination-contiguous list whose
// sources were checked pinned: the list (cut into pieces when it is short and
// its entries large) becomes the worker's next job.  Returns 0, kZcNotTaken
// (the worker is off after a failure, the destination is not device memory,
// or the list does not fit the worker's table) or an error.
int CpuPollingThread::direct_worker(const SGEntry* entries, int count, size_t total) {
    if (!worker_->ok() || count > worker_->capacity() || !zc_dst_in_device(entries[0].dst, entries[0].dst + total)) return kZcNotTaken;
    static const uint64_t timeout_us = [] {
        const char* v = std::getenv("GFD_DIRECT_TIMEOUT_MS");
        return (uint64_t)std::max(1ll, v && *v ? std::atoll(v) : 10000ll) * 1000ull;
    }();
    std::lock_guard<std::recursive_mutex> lock(worker_->mutex());
    bool cut = false;
    const int n = zc_fill_sg_table(entries, count, total, worker_->table(), worker_->capacity(), &cut,
                                   worker_->waves());
    trace(TRACE_ZC_LAUNCH, (uint32_t)count, total);
    const int rc = worker_->run(n, timeout_us);
    trace(TRACE_ZC_DONE, 0, worker_->jobs());
    return rc;
}

// The zero-copy head of a staged Direct call, planned before the gather job
// is published: the first entries, up to direct_zc_head_bytes_ bytes, when
// their sources are pinned and the destination lies in device memory.
// Returns the number of head entries (0: none; the staged route then takes
// the whole list) and their bytes.
int CpuPollingThread::zc_plan_head(const SGEntry* entries, int count, size_t total, bool uniform,
                                   size_t* head_bytes) {
    if (direct_zc_head_bytes_ == 0 || direct_zc_max_bytes_ == 0 || count < 2 || total <= direct_zc_head_bytes_)
        return 0;
    int k = 0;
    size_t bytes = 0;
    while (k < count - 1 && bytes + entries[k].size <= direct_zc_head_bytes_) bytes += entries[k++].size;
    if (k == 0 || (uniform ? !ensure_zc_src_table(k) : zc_table_cap_ < k) || !zc_ready() ||
        !zc_dst_in_device(entries[0].dst, entries[0].dst + total) || !zc_sources_pinned(entries, k, false))
        return 0;
    *head_bytes = bytes;
    return k;
}

// Launches the planned head: its address table, then the kernel.  0 or an
// error; *gen is the generation to wait for.
int CpuPollingThread::zc_launch_head(const SGEntry* entries, int k, bool uniform, uint64_t* gen) {
    const uint64_t g = ++zc_gen_;
    int rc;
    if (uniform) {
        for (int i = 0; i < k; i++) zc_src_table_[i] = (uint64_t)(uintptr_t)entries[i].src;
        rc = gfd_zero_copy_gather_tokens_signal(zc_src_table_, (void*)(uintptr_t)entries[0].dst,
                                                (uint32_t)entries[0].size, k, zc_counter_, zc_done_, g, zc_stream_);
    } else {
        size_t bytes = 0;
        for (int i = 0; i < k; i++) bytes += entries[i].size;
        bool cut = false;
        static const int kWaves = gfd_zero_copy_target_waves();
        const int n = zc_fill_sg_table(entries, k, bytes, zc_table_, zc_table_cap_, &cut, kWaves);
        rc = (cut ? gfd_zero_copy_gather_signal_presliced : gfd_zero_copy_gather_signal)(
            reinterpret_cast<const gfd_sg_entry*>(zc_table_), n, zc_counter_, zc_done_, g, zc_stream_);
    }
    if (rc != 0) return rc;
    trace(TRACE_ZC_LAUNCH, (uint32_t)k, 0);
    *gen = g;
    return 0;
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
            gather_->run(entries, count, total, direct_staging_, direct_chunk_bytes_, nullptr, nullptr,
                         uniform ? 1 : 0);
        }
        size_t off = 0;
        for (int i = 0; i < count; i++) {
            zc_table_[i] = SGEntry{entries[i].dst, direct_staging_ + off, entries[i].size};
            off += entries[i].size;
        }
    }
    if (!zc_ready()) return -1;
    const uint64_t gen = ++zc_gen_;
    int rc = gfd_zero_copy_gather_signal(reinterpret_cast<const gfd_sg_entry*>(zc_table_), count, zc_counter_,
                                         zc_done_, gen, zc_stream_);
    if (rc == 0) rc = zc_wait(gen);
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
    direct_ce_manager_.trust_range(direct_staging_, direct_staging_size_);
    if (direct_zc_max_bytes_ > 0 && !zc_warm_up()) {
        // The staged route (gather + copy engines) still serves every list.
        GFD_LOG_ERROR("zero-copy route set-up failed; submit_direct uses the copy engines only\n");
        direct_zc_max_bytes_ = 0;
    }
    if (worker_wanted_) ensure_worker();
    return start_workers();
}

double CpuPollingThread::submit_direct(const SGEntry* entries, int count) {
    if (!direct_ce_manager_.is_initialized() || count <= 0 || !entries) return -1.0;
    std::lock_guard<std::mutex> direct_lock(direct_mutex_);
    const auto t0 = std::chrono::steady_clock::now();
    if (direct_ce_manager_.pin_context() != 0) return -1.0;
    // Address ranges found pinned (sources) or in device memory (destinations)
    // by an earlier call may have been freed and reused since: look them up
    // again, once per distinct allocation, in this call.
    direct_ce_manager_.forget_pinned_range();
    zc_dst_lo_ = zc_dst_hi_ = 0;

    // Total bytes and the three list properties the route depends on (split
    // over the gather workers for long lists).
    size_t total = entries[0].size;
    bool dst_contig = true, src_contig = true, uniform = true;
    int zc_pinned = -1;  // zero-copy route: sources checked pinned and table filled (1), not pinned (0), unknown
    if (count <= GatherEngine::kCallerScanMax && direct_zc_max_bytes_ > 0 && ensure_zc_src_table(count)) {
        // Short list: one pass on this thread gives the route's properties and,
        // for the zero-copy route, the pinned check and the source table.
        // The gather workers are not woken: this route does not use them.
        bool pinned = true;
        uintptr_t lo = 1, hi = 0;
        for (int i = 0; i < count; i++) {
            const SGEntry& e = entries[i];
            if (i > 0) {
                const SGEntry& p = entries[i - 1];
                total += e.size;
                dst_contig &= e.dst == p.dst + p.size;
                src_contig &= (const char*)e.src == (const char*)p.src + p.size;
                uniform &= e.size == p.size;
            }
            const uintptr_t a = (uintptr_t)e.src, b = a + e.size;
            if (pinned && (a < lo || b > hi)) {
                pinned = direct_ce_manager_.host_source_ok(e.src, e.size);
                direct_ce_manager_.last_pinned_range(&lo, &hi);
                if (a < lo || b > hi) lo = a, hi = b;
            }
            zc_src_table_[i] = (uint64_t)a;
        }
        zc_pinned = pinned ? 1 : 0;
    } else if (gather_) {
        gather_->prewake();  // workers wake while the list is inspected
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
    if (worker_ && dst_contig && zc_pinned == 1 && total <= direct_zc_max_bytes_ &&
        (err = direct_worker(entries, count, total)) != kZcNotTaken) {
        // done by the persistent zero-copy worker (err 0) or failed
    } else if (dst_contig && src_contig) {
        err = 0;
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
    } else if (dst_contig && total <= direct_zc_max_bytes_ && total > direct_zc_min_bytes_ && count > 1 &&
               zc_pinned != 0 &&
               (err = direct_zero_copy(entries, count, total, uniform, zc_pinned == 1)) != kZcNotTaken) {
        // done by the zero-copy kernel (err 0) or failed
    } else if (dst_contig && direct_staging_ && total <= direct_staging_size_) {
        err = 0;
        std::lock_guard<std::mutex> lock(gather_mutex_);
        if (gather_) {
            // The kernel moves the head while the rest is staged.  It is
            // launched before the gather job is published: launched from
            // inside the job (once the workers have it) it measured the same
            // at 8192 x 4 KiB and 1% slower at 2048 x 64 KiB.
            size_t head_bytes = 0;
            uint64_t head_gen = 0;
            const int head = zc_plan_head(entries, count, total, uniform, &head_bytes);
            const int herr = head ? zc_launch_head(entries, head, uniform, &head_gen) : 0;
            if (herr) {
                err = herr;
            } else {
                DirectCtx ctx{this, &direct_ce_manager_, entries[head].dst, direct_staging_, nch, 0};
                gather_->run(entries + head, count - head, total - head_bytes, direct_staging_,
                             direct_chunk_bytes_, direct_chunk, &ctx, uniform ? 1 : 0);
                err = ctx.err;
                trace_gather_run();
                if (head) {
                    const int zerr = zc_wait(head_gen);
                    trace(TRACE_ZC_DONE, 0, head_gen);
                    if (zerr && !err) err = zerr;
                }
            }
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
