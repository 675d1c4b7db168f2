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

// Pause iterations an idle worker spins before it sleeps (a few hundred
// microseconds: long enough to bridge back-to-back gathers).
unsigned spin_limit() {
    const char* v = std::getenv("GFD_GATHER_SPIN");
    return (v && *v) ? (unsigned)std::strtoul(v, nullptr, 0) : 20000u;
}

}  // namespace

GatherEngine::GatherEngine(const std::vector<int>& worker_cpus) {
    wstate_.reset(new WorkerState[worker_cpus.size() ? worker_cpus.size() : 1]);
    for (size_t w = 0; w < worker_cpus.size(); w++)
        threads_.emplace_back(&GatherEngine::worker_main, this, (int)w, worker_cpus[w]);
}

GatherEngine::~GatherEngine() {
    running_.store(false, std::memory_order_seq_cst);
    epoch_.fetch_add(1, std::memory_order_seq_cst);
    futex_wake_all(&epoch_);
    for (auto& t : threads_)
        if (t.joinable()) t.join();
}

// Spin on the job counter, then sleep on it: idle workers give their cores
// back to the application and the poller instead of burning them.
void GatherEngine::worker_main(int w, int cpu) {
    if (cpu >= 0) {
        cpu_set_t cs;
        CPU_ZERO(&cs);
        CPU_SET(cpu, &cs);
        pthread_setaffinity_np(pthread_self(), sizeof(cs), &cs);
    }
    const unsigned spin = spin_limit();
    uint32_t seen = 0;
    for (;;) {
        const uint32_t e = epoch_.load(std::memory_order_acquire);
        if (!running_.load(std::memory_order_acquire)) break;
        if (e != seen) {
            seen = e;
            do_slices();
            wstate_[w].done_epoch.store(e, std::memory_order_release);
            continue;
        }
        bool moved = false;
        for (unsigned i = 0; i < spin; i++) {
            cpu_relax();
            if (epoch_.load(std::memory_order_relaxed) != seen) {
                moved = true;
                break;
            }
        }
        if (moved) continue;
        // Dekker handshake with run(): either run() sees sleepers_ > 0 and
        // wakes us, or we see the new epoch here and do not sleep.
        sleepers_.fetch_add(1, std::memory_order_seq_cst);
        if (epoch_.load(std::memory_order_seq_cst) == seen && running_.load(std::memory_order_seq_cst))
            futex_wait(&epoch_, seen);
        sleepers_.fetch_sub(1, std::memory_order_seq_cst);
    }
}

void GatherEngine::copy_slice(const Slice& s) {
    size_t left = s.len;
    int e = s.entry;
    size_t eo = s.entry_off;
    char* d = staging_ + s.off;
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
}

void GatherEngine::do_slices() {
    const int ns = (int)slices_.size();
    for (;;) {
        int s = next_slice_.fetch_add(1, std::memory_order_relaxed);
        if (s >= ns) break;
        copy_slice(slices_[s]);
        store_fence();
        remaining_[slices_[s].chunk].fetch_sub(1, std::memory_order_release);
    }
}

void GatherEngine::run(const SGEntry* entries, int count, size_t total, char* staging,
                       size_t chunk_bytes, ChunkFn on_chunk, void* ctx) {
    if (count <= 0 || total == 0) return;
    if (chunk_bytes == 0) chunk_bytes = total;
    const int nchunks = (int)((total + chunk_bytes - 1) / chunk_bytes);

    // Cut the destination stream into slices that never cross a chunk edge.
    slices_.clear();
    int e = 0;
    size_t eo = 0;
    size_t pos = 0;
    for (int c = 0; c < nchunks; c++) {
        size_t cend = std::min(total, (size_t)(c + 1) * chunk_bytes);
        while (pos < cend) {
            while (e < count && eo == entries[e].size) {  // skip spent / empty entries
                e++;
                eo = 0;
            }
            size_t len = std::min(slice_bytes_, cend - pos);
            slices_.push_back(Slice{e, eo, pos, len, c});
            size_t adv = len;
            while (adv) {
                size_t avail = entries[e].size - eo;
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
        }
    }
    if (remaining_cap_ < nchunks) {
        remaining_.reset(new std::atomic<int>[nchunks]);
        remaining_cap_ = nchunks;
    }
    for (int c = 0; c < nchunks; c++) remaining_[c].store(0, std::memory_order_relaxed);
    for (const Slice& s : slices_) remaining_[s.chunk].fetch_add(1, std::memory_order_relaxed);

    entries_ = entries;
    count_ = count;
    staging_ = staging;
    next_slice_.store(0, std::memory_order_relaxed);

    const int nw = num_workers();
    const bool caller_copy = caller_copies_ >= 0 ? (caller_copies_ != 0 || nw == 0) : (nw < 2);
    const uint32_t ep = epoch_.fetch_add(1, std::memory_order_seq_cst) + 1;
    if (sleepers_.load(std::memory_order_seq_cst) > 0) futex_wake_all(&epoch_);
    const int ns = (int)slices_.size();

    int ready = 0;
    while (ready < nchunks) {
        if (remaining_[ready].load(std::memory_order_acquire) == 0) {
            size_t off = (size_t)ready * chunk_bytes;
            size_t len = std::min(chunk_bytes, total - off);
            on_chunk(ctx, ready, off, len);
            ready++;
            continue;
        }
        if (caller_copy) {
            int s = next_slice_.fetch_add(1, std::memory_order_relaxed);
            if (s < ns) {
                copy_slice(slices_[s]);
                store_fence();
                remaining_[slices_[s].chunk].fetch_sub(1, std::memory_order_release);
                continue;
            }
        }
        cpu_relax();
    }
    for (int w = 0; w < nw; w++)
        while (wstate_[w].done_epoch.load(std::memory_order_acquire) != ep) cpu_relax();
}

}  // namespace gfd
