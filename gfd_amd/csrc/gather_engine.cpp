// Pipelined multi-threaded host gather (see gather_engine.h).
#include "gather_engine.h"

#include <immintrin.h>
#include <linux/futex.h>
#include <pthread.h>
#include <sched.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cstring>

namespace gfd {

namespace {

__attribute__((target("avx512f"))) void copy_nt_avx512(char* d, const char* s, size_t n) {
    // d is 64-byte aligned, n a multiple of 64
    size_t i = 0;
    for (; i + 256 <= n; i += 256) {
        __m512i a = _mm512_loadu_si512((const void*)(s + i));
        __m512i b = _mm512_loadu_si512((const void*)(s + i + 64));
        __m512i c = _mm512_loadu_si512((const void*)(s + i + 128));
        __m512i e = _mm512_loadu_si512((const void*)(s + i + 192));
        _mm512_stream_si512((__m512i*)(d + i), a);
        _mm512_stream_si512((__m512i*)(d + i + 64), b);
        _mm512_stream_si512((__m512i*)(d + i + 128), c);
        _mm512_stream_si512((__m512i*)(d + i + 192), e);
    }
    for (; i < n; i += 64) {
        __m512i a = _mm512_loadu_si512((const void*)(s + i));
        _mm512_stream_si512((__m512i*)(d + i), a);
    }
}

__attribute__((target("avx2"))) void copy_nt_avx2(char* d, const char* s, size_t n) {
    for (size_t i = 0; i < n; i += 64) {
        __m256i a = _mm256_loadu_si256((const __m256i*)(s + i));
        __m256i b = _mm256_loadu_si256((const __m256i*)(s + i + 32));
        _mm256_stream_si256((__m256i*)(d + i), a);
        _mm256_stream_si256((__m256i*)(d + i + 32), b);
    }
}

using CopyFn = void (*)(char*, const char*, size_t);

CopyFn pick_copy() {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f")) return copy_nt_avx512;
    return copy_nt_avx2;
}

const CopyFn g_copy_nt = pick_copy();

inline void cpu_relax() { _mm_pause(); }

}  // namespace

void stream_copy(void* dst, const void* src, size_t n) {
    char* d = (char*)dst;
    const char* s = (const char*)src;
    if (n < 256) {
        std::memcpy(d, s, n);
        return;
    }
    size_t head = (64 - ((uintptr_t)d & 63)) & 63;
    if (head) {
        std::memcpy(d, s, head);
        d += head;
        s += head;
        n -= head;
    }
    size_t body = n & ~(size_t)63;
    g_copy_nt(d, s, body);
    if (body < n) std::memcpy(d + body, s + body, n - body);
}

void store_fence() { _mm_sfence(); }

namespace {

void futex_wait(std::atomic<uint32_t>* addr, uint32_t expected) {
    syscall(SYS_futex, reinterpret_cast<uint32_t*>(addr), FUTEX_WAIT_PRIVATE, expected, nullptr, nullptr, 0);
}

void futex_wake_all(std::atomic<uint32_t>* addr) {
    syscall(SYS_futex, reinterpret_cast<uint32_t*>(addr), FUTEX_WAKE_PRIVATE, INT32_MAX, nullptr, nullptr, 0);
}

// Microseconds an idle worker spins before it sleeps: long enough to bridge
// the copy tail between back-to-back gathers (GFD_GATHER_SPIN_US).
uint64_t spin_limit_ns() {
    const char* v = std::getenv("GFD_GATHER_SPIN_US");
    const uint64_t us = (v && *v) ? (uint64_t)std::strtoull(v, nullptr, 0) : 1000u;
    return us * 1000u;
}

inline uint64_t mono_ns() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

}  // namespace

GatherEngine::GatherEngine(const std::vector<int>& worker_cpus) {
    if (const char* v = std::getenv("GFD_GATHER_PREFETCH_BYTES")) prefetch_bytes_ = std::strtoull(v, nullptr, 0);
    mail_.reset(new Mailbox[worker_cpus.empty() ? 1 : worker_cpus.size()]);
    for (size_t w = 0; w < worker_cpus.size(); w++)
        threads_.emplace_back(&GatherEngine::worker_main, this, (int)w, worker_cpus[w]);
}

GatherEngine::~GatherEngine() {
    running_.store(false, std::memory_order_seq_cst);
    const uint32_t e = epoch_.fetch_add(1, std::memory_order_seq_cst) + 1;
    for (size_t w = 0; w < threads_.size(); w++) mail_[w].go.store(e, std::memory_order_seq_cst);
    futex_wake_all(&epoch_);
    for (auto& t : threads_)
        if (t.joinable()) t.join();
}

// Job hand-off.  The caller builds the job, sets open_, takes the next job
// number, writes it to every worker's mailbox and wakes sleepers; when every
// chunk is complete it clears open_ and returns without waiting for the
// workers.  A worker that sees a new number in its mailbox raises its in_job
// flag and then checks open_; the caller rebuilds job state only after every
// in_job flag is down.  With sequentially consistent operations on open_ and
// the flags, a worker either is seen inside (and the caller waits for it) or
// sees open_ cleared and leaves without touching the job.  (Whole-list jobs
// keep their state in the mailboxes and do not come through here.)
void GatherEngine::publish() {
    open_.store(true, std::memory_order_seq_cst);
    const uint32_t e = epoch_.fetch_add(1, std::memory_order_seq_cst) + 1;
    for (size_t w = 0; w < threads_.size(); w++) mail_[w].go.store(e, std::memory_order_release);
}

void GatherEngine::wait_workers_out() {
    for (size_t w = 0; w < threads_.size(); w++)
        while (mail_[w].in_job.load(std::memory_order_seq_cst) != 0) cpu_relax();
}

void GatherEngine::worker_main(int w, int cpu) {
    if (cpu >= 0) {
        cpu_set_t cs;
        CPU_ZERO(&cs);
        CPU_SET(cpu, &cs);
        pthread_setaffinity_np(pthread_self(), sizeof(cs), &cs);
    }
    Mailbox& mb = mail_[w];
    const uint64_t spin_ns = spin_limit_ns();
    // Workers start before any job (the constructor creates them with every
    // mailbox at 0), so a job published before this thread first runs still
    // counts as new.
    uint32_t seen = 0;
    for (;;) {
        if (!running_.load(std::memory_order_acquire)) break;
        const uint32_t g = mb.go.load(std::memory_order_acquire);
        if (g != seen) {
            seen = g;
            if (mb.tag.load(std::memory_order_relaxed) == g) {  // a whole-list slice of job g
                take_mailbox_slice(mb, g, prefetch_bytes_);
                continue;
            }
            mb.in_job.store(1, std::memory_order_seq_cst);
            if (open_.load(std::memory_order_seq_cst) && running_.load(std::memory_order_relaxed)) do_job(w);
            mb.in_job.store(0, std::memory_order_seq_cst);
            continue;
        }
        bool moved = false;
        const uint64_t t_end = mono_ns() + spin_ns;
        for (unsigned i = 1;; i++) {
            cpu_relax();
            if (mb.go.load(std::memory_order_relaxed) != seen) {
                moved = true;
                break;
            }
            if ((i & 255) == 0 && mono_ns() >= t_end) break;
        }
        if (moved) continue;
        // Dekker handshake with publish() and run_whole() (each stores go,
        // then bumps epoch_ with a full fence, then reads sleepers_): either
        // the caller sees sleepers_ > 0 and wakes us after the bump, or we see
        // the new job here and do not sleep.  futex_wait returns at once if
        // epoch_ has moved on.
        sleepers_.fetch_add(1, std::memory_order_seq_cst);
        const uint32_t e = epoch_.load(std::memory_order_seq_cst);
        if (mb.go.load(std::memory_order_seq_cst) == seen && running_.load(std::memory_order_seq_cst))
            futex_wait(&epoch_, e);
        sleepers_.fetch_sub(1, std::memory_order_seq_cst);
    }
}

void GatherEngine::prewake() {
    last_prewake_ns_.store(mono_ns(), std::memory_order_relaxed);
    if (sleepers_.load(std::memory_order_seq_cst) > 0) futex_wake_all(&epoch_);
}

namespace {

// Copy `left` bytes of the list, starting at byte eo of entry e, to d.
void copy_span(const SGEntry* entries_, int count_, int e, size_t eo, char* d, size_t left,
               size_t prefetch_bytes) {
    // Source prefetch runs kPrefetchAhead bytes of this slice ahead of the
    // copy, every line of each token it passes (scattered small tokens miss
    // in cache on every line; one line per token left 512 B tokens latency
    // bound).  Tokens longer than kPrefetchLines lines get their first lines
    // only: the hardware stream prefetcher covers the rest.
    const size_t kPrefetchAhead = prefetch_bytes;
    constexpr size_t kPrefetchLines = 16;
    if (kPrefetchAhead == 0) {  // one line of the token four entries ahead
        while (left) {
            size_t avail = entries_[e].size - eo;
            size_t n = avail < left ? avail : left;
            if (n) {
                if (e + 4 < count_) __builtin_prefetch(entries_[e + 4].src, 0, 0);
                stream_copy(d, (const char*)entries_[e].src + eo, n);
                d += n;
                left -= n;
            }
            e++;
            eo = 0;
        }
        return;
    }
    int pe = e;
    size_t po = eo, pahead = 0;  // prefetch cursor (entry, offset) and its lead in bytes
    auto advance_prefetch = [&](size_t target) {
        while (pahead < target && pe < count_) {
            const size_t sz = entries_[pe].size;
            const char* p = (const char*)entries_[pe].src;
            const size_t lim = std::min(sz, kPrefetchLines * 64);
            for (size_t o = po & ~(size_t)63; o < lim; o += 64) __builtin_prefetch(p + o, 0, 3);
            pahead += sz - po;
            po = 0;
            pe++;
        }
    };
    advance_prefetch(std::min(kPrefetchAhead, left));
    while (left) {
        size_t avail = entries_[e].size - eo;
        size_t n = avail < left ? avail : left;
        if (n) {
            stream_copy(d, (const char*)entries_[e].src + eo, n);
            d += n;
            left -= n;
            pahead = pahead > n ? pahead - n : 0;
            if (left) advance_prefetch(std::min(kPrefetchAhead, left));
        }
        e++;
        eo = 0;
    }
}

}  // namespace

void GatherEngine::copy_slice(const Slice& s) {
    copy_span(entries_, count_, s.entry, s.entry_off, staging_ + s.off, s.len, prefetch_bytes_);
}

void GatherEngine::do_job(int w) {
    if (scan_job_) do_scan_parts();
    else do_slices();
}

// Whole-list job: take the slice described in mb if job `job` is still open
// there (nobody has claimed it for this job), copy it and mark it done.
bool GatherEngine::take_mailbox_slice(Mailbox& mb, uint32_t job, size_t prefetch_bytes) {
    uint32_t c = mb.claimed.load(std::memory_order_relaxed);
    for (;;) {
        if ((int32_t)(job - c) <= 0) return false;  // taken for this job (or a later one)
        if (mb.claimed.compare_exchange_weak(c, job, std::memory_order_acq_rel, std::memory_order_relaxed)) break;
    }
    copy_span(mb.entries, mb.count, mb.entry, mb.entry_off, mb.dst, mb.len, prefetch_bytes);
    store_fence();
    mb.done.store(job, std::memory_order_release);
    return true;
}

// Scan job: claim parts of kScanPartEntries entries; part k checks the pairs
// (i-1, i) for i in its range, so every adjacent pair is checked once.  The
// list is read only after a claim: a worker can reach this loop just as the
// caller, having seen every part done, returns and the list is freed.
void GatherEngine::do_scan_parts() {
    const SGEntry* e = entries_;
    for (;;) {
        const int k = next_slice_.fetch_add(1, std::memory_order_relaxed);
        if (k >= scan_parts_) break;
        const size_t size0 = e[0].size;
        const int b = k * kScanPartEntries, end = std::min(count_, b + kScanPartEntries);
        size_t sum = 0;
        bool dc = true, sc = true, un = true;
        for (int i = b; i < end; i++) {
            sum += e[i].size;
            un &= e[i].size == size0;
            if (i > 0) {
                dc &= e[i].dst == e[i - 1].dst + e[i - 1].size;
                sc &= (const char*)e[i].src == (const char*)e[i - 1].src + e[i - 1].size;
            }
        }
        ScanPart& o = scan_out_[k];
        o.sum = sum;
        o.dst_contig = dc;
        o.src_contig = sc;
        o.uniform = un;
        scan_left_.fetch_sub(1, std::memory_order_release);
    }
}

GatherEngine::ListScan GatherEngine::scan(const SGEntry* entries, int count) {
    ListScan r{0, true, true, true};
    if (count <= 0) return r;
    if (count <= kCallerScanMax || threads_.empty()) {
        r.total = entries[0].size;
        for (int i = 1; i < count; i++) {
            const SGEntry& p = entries[i - 1];
            const SGEntry& e = entries[i];
            r.total += e.size;
            r.dst_contig &= e.dst == p.dst + p.size;
            r.src_contig &= (const char*)e.src == (const char*)p.src + p.size;
            r.uniform &= e.size == p.size;
        }
        return r;
    }
    wait_workers_out();
    entries_ = entries;
    count_ = count;
    scan_parts_ = (count + kScanPartEntries - 1) / kScanPartEntries;
    if ((int)scan_out_.size() < scan_parts_) scan_out_.resize(scan_parts_);
    scan_left_.store(scan_parts_, std::memory_order_relaxed);
    next_slice_.store(0, std::memory_order_relaxed);
    scan_job_ = true;
    publish();
    if (sleepers_.load(std::memory_order_seq_cst) > 0 && mono_ns() - last_prewake_ns_.load(std::memory_order_relaxed) > 200000ull)
        futex_wake_all(&epoch_);
    do_scan_parts();
    while (scan_left_.load(std::memory_order_acquire) != 0) cpu_relax();
    open_.store(false, std::memory_order_seq_cst);
    for (int k = 0; k < scan_parts_; k++) {
        const ScanPart& o = scan_out_[k];
        r.total += o.sum;
        r.dst_contig &= o.dst_contig;
        r.src_contig &= o.src_contig;
        r.uniform &= o.uniform;
    }
    // The next run() waits for the workers to leave before reusing job state.
    return r;
}

int GatherEngine::chunk_of(int s) const {
    if (!lazy_) return slices_[s].chunk;
    int lo = 0, hi = (int)chunk_first_.size() - 1;  // chunk_first_ is strictly increasing
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (chunk_first_[mid] <= s) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

GatherEngine::Slice GatherEngine::slice_at(int s) const {
    if (!lazy_) return slices_[s];
    const int c = chunk_of(s);
    const size_t sb = chunk_slice_[c];
    const size_t pos = (c ? chunk_end_[c - 1] : 0) + (size_t)(s - chunk_first_[c]) * sb;
    const size_t len = std::min(sb, chunk_end_[c] - pos);
    return Slice{(int)(pos / esz_), pos % esz_, pos, len, c};
}

// Claim and copy slices until none are left.  Returns after the last claim.
void GatherEngine::do_slices() {
    const int ns = num_slices_;
    bool counted = false;
    for (;;) {
        const int s = next_slice_.fetch_add(1, std::memory_order_relaxed);
        if (s >= ns) break;
        const Slice sl = slice_at(s);
        copy_slice(sl);
        store_fence();
        note_slice(counted);
        remaining_[sl.chunk].fetch_sub(1, std::memory_order_release);
    }
}

void GatherEngine::note_slice(bool& counted) {
    if (counted) return;
    counted = true;
    copiers_.fetch_add(1, std::memory_order_relaxed);
    uint64_t z = 0;
    first_slice_ns_.compare_exchange_strong(z, mono_ns(), std::memory_order_relaxed);
}

void GatherEngine::run(const SGEntry* entries, int count, size_t total, char* staging,
                       size_t chunk_bytes, ChunkFn on_chunk, void* ctx, int uniform_hint) {
    if (count <= 0 || total == 0) return;
    if (on_chunk == nullptr) {
        run_whole(entries, count, total, staging, uniform_hint);
        return;
    }
    times_.entry = mono_ns();
    if (chunk_bytes == 0 || chunk_bytes > total) chunk_bytes = total;
    // Workers still inside the previous job must leave before its state changes.
    wait_workers_out();
    times_.idle = mono_ns();
    first_slice_ns_.store(0, std::memory_order_relaxed);
    copiers_.store(0, std::memory_order_relaxed);

    // Chunk edges: a short first chunk gets the first copy going early; with
    // the ramp on, each following chunk doubles until chunk_bytes, so every
    // chunk is gathered before the copies ahead of it drain and the host
    // link never waits for the next chunk (the threads gather faster than
    // the link drains).
    size_t first = first_chunk_bytes_ ? first_chunk_bytes_ : chunk_bytes / 8;
    if (first < 64 * 1024) first = 64 * 1024;
    if (first > chunk_bytes) first = chunk_bytes;

    chunk_end_.clear();
    size_t size = first;
    for (size_t end = first;;) {
        chunk_end_.push_back(std::min(end, total));
        if (end >= total) break;
        size = ramp_ ? std::min(size * 2, chunk_bytes) : chunk_bytes;
        end += size;
    }
    const int nchunks = (int)chunk_end_.size();

    // Cut the destination stream into slices that never cross a chunk edge.
    // The first chunk uses finer slices so every thread shares it and the
    // first copy starts as early as possible.
    const size_t esz = entries[0].size;
    bool uniform = uniform_hint > 0;
    if (uniform_hint < 0) {
        uniform = true;
        for (int i = 1; i < count && uniform; i++) uniform = entries[i].size == esz;
    }
    uniform = uniform && esz > 0;
    // Slices: about two per thread for the whole job, between 16 KiB and
    // slice_bytes_.  A small job (a 0.5 MiB queue batch) cut into 128 KiB
    // slices leaves a whole chunk to one thread while the others idle.
    const size_t threads = (size_t)num_workers() + 1;
    const size_t job_slice = std::max<size_t>(
        16 * 1024, std::min(slice_bytes_, ((total / (2 * threads)) + 4095) & ~(size_t)4095));
    const size_t first_slice = std::max<size_t>(16 * 1024, std::min(job_slice, chunk_end_[0] / 16));
    if (remaining_cap_ < nchunks) {
        remaining_.reset(new std::atomic<int>[nchunks]);
        remaining_cap_ = nchunks;
    }
    lazy_ = uniform;
    int nslices = 0;
    if (uniform) {
        // Slice s of chunk c starts (s - chunk_first_[c]) slices into it.
        esz_ = esz;
        chunk_first_.resize(nchunks);
        chunk_slice_.resize(nchunks);
        size_t start = 0;
        for (int c = 0; c < nchunks; c++) {
            const size_t sb = c == 0 ? first_slice : job_slice;
            const int k = (int)((chunk_end_[c] - start + sb - 1) / sb);
            chunk_first_[c] = nslices;
            chunk_slice_[c] = sb;
            remaining_[c].store(k, std::memory_order_relaxed);
            nslices += k;
            start = chunk_end_[c];
        }
    } else {
        slices_.clear();
        int e = 0;
        size_t eo = 0;
        size_t pos = 0;
        for (int c = 0; c < nchunks; c++) {
            const size_t cend = chunk_end_[c];
            const size_t sb = c == 0 ? first_slice : job_slice;
            int k = 0;
            while (pos < cend) {
                const size_t len = std::min(sb, cend - pos);
                while (e < count && eo == entries[e].size) {  // skip spent / empty entries
                    e++;
                    eo = 0;
                }
                slices_.push_back(Slice{e, eo, pos, len, c});
                size_t adv = len;
                while (adv) {
                    const size_t avail = entries[e].size - eo;
                    if (avail > adv) {
                        eo += adv;
                        adv = 0;
                    } else {
                        adv -= avail;
                        e++;
                        eo = 0;
                    }
                }
                pos += len;
                k++;
            }
            remaining_[c].store(k, std::memory_order_relaxed);
        }
        nslices = (int)slices_.size();
    }

    entries_ = entries;
    count_ = count;
    staging_ = staging;
    num_slices_ = nslices;
    next_slice_.store(0, std::memory_order_relaxed);
    scan_job_ = false;

    // The caller copies slices too: workers are helpers (one that is asleep
    // or late sits the job out), so the caller alone can always finish it.
    const int nw = num_workers();
    times_.built = mono_ns();
    publish();
    times_.sleepers = sleepers_.load(std::memory_order_seq_cst);
    // Workers are helpers: the caller can finish the job alone.  If they were
    // woken just before (prewake), do not pay for a second wake syscall here;
    // a worker that fell asleep in between simply sits this job out.
    if (times_.sleepers > 0 && times_.built - last_prewake_ns_.load(std::memory_order_relaxed) > 200000ull) futex_wake_all(&epoch_);
    const int ns = num_slices_;
    times_.published = mono_ns();
    bool counted = false;

    int ready = 0;
    while (ready < nchunks) {
        if (remaining_[ready].load(std::memory_order_acquire) == 0) {
            const size_t off = ready ? chunk_end_[ready - 1] : 0;
            on_chunk(ctx, ready, off, chunk_end_[ready] - off);
            ready++;
            continue;
        }
        // The caller only takes slices of the chunk it is waiting to hand
        // off: a slice of a later chunk (up to 128 KiB, ~10 us) would delay
        // the hand-off of this one by that long.  With no such slice left it
        // spins until the workers finish the chunk.
        const int peek = next_slice_.load(std::memory_order_relaxed);
        if (nw == 0 || (peek < ns && chunk_of(peek) <= ready)) {
            const int s = next_slice_.fetch_add(1, std::memory_order_relaxed);
            if (s < ns) {
                const Slice sl = slice_at(s);
                copy_slice(sl);
                store_fence();
                note_slice(counted);
                remaining_[sl.chunk].fetch_sub(1, std::memory_order_release);
                continue;
            }
        }
        cpu_relax();
    }
    open_.store(false, std::memory_order_seq_cst);
    times_.first_slice = first_slice_ns_.load(std::memory_order_relaxed);
    times_.copiers = copiers_.load(std::memory_order_relaxed);
}

// No copy to pipeline: num_workers() + 1 equal slices of 64-byte multiples,
// the static split of the reference's parallel_gather
// (src/parallel_gather.cpp:90-116), the caller's first.  Each worker finds
// its slice in its mailbox; the caller copies its own, takes any slice whose
// worker has not claimed it yet (a worker that is late or asleep leaves its
// share to the caller) and returns once every slice is written and fenced.
void GatherEngine::run_whole(const SGEntry* entries, int count, size_t total, char* staging, int uniform_hint) {
    const int nw = num_workers();
    const size_t threads = (size_t)nw + 1;
    const size_t slice = (((total + threads - 1) / threads) + 63) & ~(size_t)63;
    const int ns = (int)((total + slice - 1) / slice);  // at most threads
    const size_t esz = entries[0].size;
    bool uniform = uniform_hint > 0;
    if (uniform_hint < 0) {
        uniform = true;
        for (int i = 1; i < count && uniform; i++) uniform = entries[i].size == esz;
    }
    uniform = uniform && esz > 0;
    // Only this thread bumps epoch_ (after its own slice, below).
    const uint32_t job = epoch_.load(std::memory_order_relaxed) + 1;
    // (e, eo): the list position of byte pos.  Uniform lists step by whole
    // slices (a slice is q entries and r bytes); ragged ones walk the sizes.
    int e = 0;
    size_t eo = 0, pos = 0;
    const size_t q = uniform ? slice / esz : 0, r = uniform ? slice % esz : 0;
    for (int s = 1; s < ns; s++) {
        const size_t off = (size_t)s * slice;
        if (uniform) {
            e += (int)q;
            eo += r;
            if (eo >= esz) {
                eo -= esz;
                e++;
            }
        } else {
            while (pos < off) {
                const size_t adv = std::min(entries[e].size - eo, off - pos);
                eo += adv;
                pos += adv;
                if (eo == entries[e].size) {
                    e++;
                    eo = 0;
                }
            }
            while (e < count && eo == entries[e].size) {  // skip empty entries
                e++;
                eo = 0;
            }
        }
        // Fields, tag and go share the line: the worker can start on it as
        // soon as this line reaches it, while the next ones are written.
        Mailbox& mb = mail_[s - 1];
        mb.entries = entries;
        mb.count = count;
        mb.entry = e;
        mb.entry_off = eo;
        mb.dst = staging + off;
        mb.len = std::min(slice, total - off);
        mb.tag.store(job, std::memory_order_relaxed);
        mb.go.store(job, std::memory_order_release);
    }
    for (int w = ns - 1; w < nw; w++) mail_[w].go.store(job, std::memory_order_release);
    // Sleeping workers are woken now if there are any, so they can still
    // help; otherwise the job counter is bumped after the caller's slice,
    // where the full fence it implies (the other half of the handshake with a
    // worker about to sleep) no longer holds back the caller's first copy.
    // A worker that falls asleep in between is woken then, and its slice is
    // the caller's to take.
    bool bumped = false;
    if (sleepers_.load(std::memory_order_relaxed) > 0) {
        epoch_.fetch_add(1, std::memory_order_seq_cst);
        bumped = true;
        if (mono_ns() - last_prewake_ns_.load(std::memory_order_relaxed) > 200000ull) futex_wake_all(&epoch_);
    }
    copy_span(entries, count, 0, 0, staging, std::min(slice, total), prefetch_bytes_);
    store_fence();
    if (!bumped) {
        epoch_.fetch_add(1, std::memory_order_seq_cst);
        if (sleepers_.load(std::memory_order_seq_cst) > 0) futex_wake_all(&epoch_);
    }
    for (int s = 1; s < ns; s++) take_mailbox_slice(mail_[s - 1], job, prefetch_bytes_);
    for (int s = 1; s < ns; s++)
        while (mail_[s - 1].done.load(std::memory_order_acquire) != job) cpu_relax();
}

}  // namespace gfd
