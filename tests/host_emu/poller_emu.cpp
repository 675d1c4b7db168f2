// Runs the product poller (CpuPollingThread with its SDMA copy queue) on the
// host against the emulated runtime of emu.h, driven by threads that follow
// the device protocols of the kernels in gfd_amd/csrc/kernels:
//
//   sg <case> <rounds> <seed>
//       SG mode (set_sg_task_queue; src/batch_processor.cpp:307-446 of the
//       reference): one producer per list claims ring slots, writes the
//       list's descriptors tagged list_id << 32 | i with FLAG_LAST_IN_TILE on
//       the last, commits them, waits for d_list_done[list_id] and then
//       checksums what landed (sg_poller_kernel's protocol).  Cases:
//       split_small_tokens, ragged, host_flags, one_entry_lists, pages.
//   queue <n> <token_bytes> <scattered 0|1> <rounds> <seed>
//       Queue mode (src/cpu_polling.cpp:337-490, examples/04_benchmark.cu:
//       31-54 of the reference): producers of 256 descriptors each, the last
//       flagged FLAG_LAST_IN_BATCH, then a wait for done_idx.
//   tiled <tiles> <T> <C> <token_bytes> <whole 0|1> <hbm 0|1> <rounds> <seed>
//       Tiled mode, per-tile cumulative progress words.
//   ragged <direct|queue> <n> <runs> <rounds> <seed>
//       Ragged entries over a few destination runs, at every alignment.
//   sdma_slot_reuse
//       SdmaQueue alone: a signal slot comes round again while a copy that
//       depends on its previous occupant is still queued (see the function).
//   staging_pool <rounds> <seed>
//       StagingPool selection, acquire / release / too small, and Queue
//       pollers on pool sets and on their own staging.
//   locked_source
//       SdmaQueue::host_source_ok on registered host memory.
//   gather_mix <workers> <rounds> <seed>
//       GatherEngine alone: whole-list runs (no chunk callback), pipelined
//       runs and parallel list scans in random order on one engine (see the
//       function).
//
// Every landed byte is compared with the expected image (the entries applied
// by plain memcpy), and list checksums exactly.  Exit status: 0 pass,
// 2 a wait timed out, 3 mismatch, 4 setup failure, 86 the emulated copy
// engines stalled on each other.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "gfd/cpu_polling.h"
#include "gfd/descriptor_queue.h"
#include "emu.h"
#include "gfd/hip_shim.h"
#include "gfd/sg_task_queue.h"
#include "gfd/staging_pool.h"
#include "gfd/tiled_queue.h"
#include "gather_engine.h"
#include "sdma.h"

using namespace gfd;

namespace {

constexpr uint8_t kSentinel = 0xCD;
constexpr double kWaitSeconds = 20.0;

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed ? seed : 0x9E3779B97F4A7C15ull) {}
    uint64_t next() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    }
    uint64_t below(uint64_t n) { return next() % n; }
};

struct Entry {
    uint64_t src, dst;
    uint32_t size;
};

void* host_alloc(size_t n) {
    void* p = nullptr;
    if (gfd_hip_host_alloc(&p, n, GFD_HOST_COHERENT) != 0) {
        std::fprintf(stderr, "host alloc failed\n");
        std::exit(4);
    }
    return p;
}

void* dev_alloc(size_t n) {
    void* p = nullptr;
    if (gfd_hip_malloc(&p, n) != 0) {
        std::fprintf(stderr, "device alloc failed\n");
        std::exit(4);
    }
    return p;
}

double seconds_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

uint64_t word_checksum(const uint8_t* p, uint32_t n) {
    uint64_t acc = 0;
    const uint32_t nw = n / 4;
    for (uint32_t k = 0; k < nw; k++) {
        uint32_t w;
        std::memcpy(&w, p + 4 * k, 4);
        acc += w;
    }
    for (uint32_t b = nw * 4; b < n; b++) acc += p[b];
    return acc;
}

// Claim `count` consecutive ring slots and commit descriptors for them; lanes
// of a wave commit in no fixed order, so each group of 64 is committed in a
// shuffled order.
uint64_t post(DescriptorQueue* q, const Entry* e, uint32_t count, uint64_t tag_hi, uint32_t last_flag, Rng& rng) {
    const uint64_t base = __atomic_fetch_add(&q->write_idx, (uint64_t)count, __ATOMIC_RELAXED);
    uint32_t order[64];
    for (uint32_t g = 0; g < count; g += 64) {
        const uint32_t n = std::min<uint32_t>(64, count - g);
        for (uint32_t k = 0; k < n; k++) order[k] = k;
        for (uint32_t k = n; k > 1; k--) std::swap(order[k - 1], order[rng.below(k)]);
        for (uint32_t k = 0; k < n; k++) {
            const uint32_t i = g + order[k];
            Descriptor* d = &q->entries[(base + i) % QUEUE_SIZE];
            d->src_addr = e[i].src;
            d->dst_addr = e[i].dst;
            d->size = e[i].size;
            d->flags = i == count - 1 ? last_flag : FLAG_NONE;
            d->user_data = (tag_hi << 32) | i;
            __atomic_store_n(&d->sequence, base + i + 1, __ATOMIC_RELEASE);
        }
    }
    return base;
}

bool wait_u64(volatile uint64_t* p, uint64_t at_least) {
    const auto t0 = std::chrono::steady_clock::now();
    while (__atomic_load_n(p, __ATOMIC_ACQUIRE) < at_least) {
        if (seconds_since(t0) > kWaitSeconds) return false;
        std::this_thread::yield();
    }
    return true;
}

int check_image(const uint8_t* got, const std::vector<uint8_t>& want, const char* what, int rnd) {
    size_t bad = 0, first = 0;
    for (size_t i = 0; i < want.size(); i++)
        if (got[i] != want[i]) {
            if (!bad) first = i;
            bad++;
        }
    if (bad) {
        std::printf("%s round %d: %zu mismatched bytes (first at %zu)\n", what, rnd, bad, first);
        return 3;
    }
    return 0;
}

int run_sg(const std::string& kase, int rounds, uint64_t seed) {
    Rng rng(seed);
    const size_t host_bytes = 8u << 20, dst_bytes = 96u << 20;
    auto* host = (uint8_t*)host_alloc(host_bytes);
    for (size_t i = 0; i < host_bytes; i++) host[i] = (uint8_t)rng.next();
    auto* dst = (uint8_t*)dev_alloc(dst_bytes);

    std::vector<uint32_t> sizes;
    uint32_t lo = 1024, hi = 1024;
    if (kase == "split_small_tokens") {
        sizes = {1500, 700, 2500, 1, 3000};
    } else if (kase == "ragged" || kase == "host_flags") {
        for (int l = 0; l < 40; l++) sizes.push_back(1 + (uint32_t)rng.below(199));
        lo = 1;
        hi = 8999;
    } else if (kase == "one_entry_lists") {
        sizes.assign(300, 1);
        lo = hi = 4096;
    } else if (kase == "pages") {
        // Page-aligned 4 KiB entries into page slots scattered over twice the
        // region, posted by one producer in list order; two lists are longer
        // than the 4096-entry batch threshold.
        sizes = {5000, 300, 1, 4500, 64};
        lo = hi = 4096;
    } else {
        std::fprintf(stderr, "unknown case %s\n", kase.c_str());
        return 4;
    }
    const bool pages = kase == "pages";
    std::vector<Entry> ent;
    std::vector<uint32_t> offs{0};
    size_t off = 0;
    std::vector<uint64_t> slot;
    if (pages) {
        size_t total = 0;
        for (uint32_t k : sizes) total += k;
        slot.resize(2 * total);
        for (size_t i = 0; i < slot.size(); i++) slot[i] = i;
        for (size_t i = slot.size(); i > 1; i--) std::swap(slot[i - 1], slot[rng.below(i)]);
        off = 2 * total * 4096;
    }
    for (uint32_t k : sizes) {
        for (uint32_t i = 0; i < k; i++) {
            const uint32_t n = lo + (uint32_t)rng.below(hi - lo + 1);
            if (pages) {
                const uint64_t so = rng.below(host_bytes / 4096) * 4096;
                const uint64_t dofs = slot[ent.size()] * 4096;
                ent.push_back(Entry{(uint64_t)(uintptr_t)host + so, (uint64_t)(uintptr_t)dst + dofs, n});
                continue;
            }
            const uint64_t so = rng.below(host_bytes - n);
            ent.push_back(Entry{(uint64_t)(uintptr_t)host + so, (uint64_t)(uintptr_t)dst + off, n});
            off += n + rng.below(33);
        }
        offs.push_back((uint32_t)ent.size());
    }
    if (off > dst_bytes) return 4;
    std::vector<uint64_t> want_sums(sizes.size(), 0);
    std::vector<uint8_t> want(off, kSentinel);
    for (size_t l = 0; l < sizes.size(); l++)
        for (uint32_t i = offs[l]; i < offs[l + 1]; i++) {
            const Entry& e = ent[i];
            want_sums[l] += word_checksum((const uint8_t*)(uintptr_t)e.src, e.size);
            std::memcpy(&want[e.dst - (uint64_t)(uintptr_t)dst], (const void*)(uintptr_t)e.src, e.size);
        }

    auto* q = (DescriptorQueue*)host_alloc(sizeof(DescriptorQueue));
    auto* sq = (SGTaskQueue*)host_alloc(sizeof(SGTaskQueue));
    const size_t flag_words = MAX_SG_LISTS + SG_DEVICE_COUNTER_WORDS;
    const bool device_flags = kase != "host_flags";
    sq->d_list_done = (uint64_t*)(device_flags ? dev_alloc(flag_words * 8) : host_alloc(flag_words * 8));

    int rc = 0;
    {
        CpuPollingThread p(q, dst, host, host_bytes, true, -1);
        p.set_sg_task_queue(sq);
        if (!p.init_copy_engine()) return 4;
        p.start();
        for (int rnd = 0; rnd < rounds && rc == 0; rnd++) {
            std::printf("sg %s round %d: %zu lists, %zu entries\n", kase.c_str(), rnd, sizes.size(), ent.size());
            std::fflush(stdout);
            std::memset(dst, kSentinel, off);
            std::memset(sq->d_list_done, 0, flag_words * 8);
            // The previous round's count is complete (checked below), so
            // the poller adds nothing more to it.
            __atomic_store_n(&sq->lists_completed, 0ull, __ATOMIC_RELAXED);
            std::vector<uint64_t> sums(sizes.size(), 0);
            std::atomic<int> timed_out{-1};
            std::vector<std::thread> wg;
            if (pages) {
                Rng lr(seed + (uint64_t)rnd);
                for (size_t l = 0; l < sizes.size(); l++)
                    post(q, &ent[offs[l]], offs[l + 1] - offs[l], l, FLAG_LAST_IN_TILE, lr);
            }
            for (size_t l = 0; l < sizes.size(); l++)
                wg.emplace_back([&, l] {
                    Rng lr(seed * 1000003u + l * 7919u + (uint64_t)rnd);
                    const uint32_t count = offs[l + 1] - offs[l];
                    if (count == 0) return;
                    if (!pages) post(q, &ent[offs[l]], count, l, FLAG_LAST_IN_TILE, lr);
                    if (!wait_u64(&sq->d_list_done[l], 1)) {
                        timed_out = (int)l;
                        return;
                    }
                    uint64_t acc = 0;
                    for (uint32_t i = offs[l]; i < offs[l + 1]; i++)
                        acc += word_checksum((const uint8_t*)(uintptr_t)ent[i].dst, ent[i].size);
                    sums[l] = acc;
                });
            for (auto& t : wg) t.join();
            if (timed_out >= 0) {
                std::printf("sg %s round %d: list %d wait timed out\n", kase.c_str(), rnd, timed_out.load());
                rc = 2;
                break;
            }
            rc = check_image(dst, want, "sg", rnd);
            for (size_t l = 0; l < sizes.size() && rc == 0; l++)
                if (sums[l] != want_sums[l]) {
                    std::printf("sg %s round %d: list %zu checksum\n", kase.c_str(), rnd, l);
                    rc = 3;
                }
            // lists_completed is raised when a list's completion point
            // retires, possibly after its flag: every list of the round,
            // once each (an empty list is never posted).
            size_t posted = 0;
            for (size_t l = 0; l < sizes.size(); l++) posted += offs[l + 1] > offs[l];
            if (rc == 0 && (!wait_u64(&sq->lists_completed, posted) ||
                            __atomic_load_n(&sq->lists_completed, __ATOMIC_ACQUIRE) != posted)) {
                std::printf("sg %s round %d: lists_completed %llu, want %zu\n", kase.c_str(), rnd,
                            (unsigned long long)__atomic_load_n(&sq->lists_completed, __ATOMIC_ACQUIRE), posted);
                rc = 5;
            }
        }
        p.stop();
    }
    if (rc == 0 && q->done_idx != (uint64_t)rounds * ent.size()) {
        std::printf("done_idx %llu, want %llu\n", (unsigned long long)q->done_idx,
                    (unsigned long long)rounds * ent.size());
        rc = 3;
    }
    if (rc == 0) std::printf("sg %s: pass\n", kase.c_str());
    gfd_hip_free(device_flags ? (void*)sq->d_list_done : nullptr);
    if (!device_flags) gfd_hip_host_free(sq->d_list_done);
    gfd_hip_host_free(sq);
    gfd_hip_host_free(q);
    gfd_hip_free(dst);
    gfd_hip_host_free(host);
    return rc;
}

// One Queue round on a started poller: producers of 256 descriptors each,
// the last flagged FLAG_LAST_IN_BATCH, then a wait for done_idx and a check
// of every byte of the destination region.
int queue_round(DescriptorQueue* q, const std::vector<Entry>& ent, uint8_t* dst, const std::vector<uint8_t>& want,
                uint64_t seed, int rnd, const char* what) {
    const uint32_t n = (uint32_t)ent.size();
    std::memset(dst, kSentinel, want.size());
    const uint64_t start = q->write_idx;
    std::vector<std::thread> wg;
    for (uint32_t b = 0; b < n; b += 256)
        wg.emplace_back([&, b] {
            Rng lr(seed + b + (uint64_t)rnd * 65537u);
            const uint32_t c = std::min<uint32_t>(256, n - b);
            post(q, &ent[b], c, 0, b + c == n ? FLAG_LAST_IN_BATCH : FLAG_NONE, lr);
        });
    for (auto& th : wg) th.join();
    if (!wait_u64(&q->done_idx, start + n)) {
        std::printf("%s round %d: done_idx wait timed out\n", what, rnd);
        return 2;
    }
    return check_image(dst, want, what, rnd);
}

int run_queue(uint32_t n, uint32_t t, bool scattered, int rounds, uint64_t seed) {
    Rng rng(seed);
    const size_t host_bytes = (size_t)n * 2 * t;
    auto* host = (uint8_t*)host_alloc(host_bytes);
    for (size_t i = 0; i < host_bytes; i++) host[i] = (uint8_t)rng.next();
    std::vector<uint32_t> perm(n);
    for (uint32_t i = 0; i < n; i++) perm[i] = i;
    for (uint32_t i = n; i > 1; i--) std::swap(perm[i - 1], perm[rng.below(i)]);
    std::vector<Entry> ent(n);
    size_t off = 0;
    auto* dst = (uint8_t*)dev_alloc((size_t)n * (t + 32) + 64);
    for (uint32_t j = 0; j < n; j++) {
        ent[j] = Entry{(uint64_t)(uintptr_t)host + (uint64_t)perm[j] * 2 * t, (uint64_t)(uintptr_t)dst + off, t};
        off += t + (scattered ? rng.below(33) : 0);
    }
    std::vector<uint8_t> want(off, kSentinel);
    for (const Entry& e : ent)
        std::memcpy(&want[e.dst - (uint64_t)(uintptr_t)dst], (const void*)(uintptr_t)e.src, e.size);
    auto* q = (DescriptorQueue*)host_alloc(sizeof(DescriptorQueue));
    int rc = 0;
    {
        CpuPollingThread p(q, dst, host, host_bytes, true, -1);
        if (!p.init_copy_engine()) return 4;
        p.start();
        for (int rnd = 0; rnd < rounds && rc == 0; rnd++) {
            std::printf("queue %ux%u scattered=%d round %d\n", n, t, (int)scattered, rnd);
            std::fflush(stdout);
            rc = queue_round(q, ent, dst, want, seed, rnd, "queue");
        }
        p.stop();
        std::printf("zero-copy worker jobs: %llu\n", (unsigned long long)p.zero_copy_worker_jobs());
    }
    if (rc == 0) std::printf("queue %ux%u scattered=%d: pass\n", n, t, (int)scattered);
    gfd_hip_host_free(q);
    gfd_hip_free(dst);
    gfd_hip_host_free(host);
    return rc;
}

// Ragged entries (1..8999 bytes, random pinned sources) whose destinations
// follow the list order, cut into `nruns` runs by odd-length gaps.  Direct:
// one submit_direct call (runs <= 64 take the staged routes); Queue: one
// producer posts the list, last entry FLAG_LAST_IN_BATCH, then a wait on
// done_idx.
int run_ragged(const std::string& path, uint32_t n, uint32_t nruns, int rounds, uint64_t seed) {
    Rng rng(seed);
    std::vector<uint32_t> sizes(n);
    size_t total = 0;
    // Entry sizes 1 .. GFD_EMU_MAX_ENTRY bytes (8999 unless set).
    const char* me = std::getenv("GFD_EMU_MAX_ENTRY");
    const uint32_t max_entry = me && *me ? (uint32_t)std::strtoul(me, nullptr, 10) : 8999u;
    for (auto& s : sizes) {
        s = 1 + (uint32_t)rng.below(max_entry);
        total += s;
    }
    const size_t host_bytes = 2 * total + 64;
    auto* host = (uint8_t*)host_alloc(host_bytes);
    for (size_t i = 0; i < host_bytes; i++) host[i] = (uint8_t)rng.next();
    std::vector<uint8_t> cut(n, 0);
    for (uint32_t k = 1; k < nruns && k < n; k++) {
        uint32_t c;
        do c = 1 + (uint32_t)rng.below(n - 1);
        while (cut[c]);
        cut[c] = 1;
    }
    std::vector<Entry> ent(n);
    size_t off = 0;
    auto* dst = (uint8_t*)dev_alloc(total + (size_t)nruns * 4200 + 4096);
    for (uint32_t i = 0; i < n; i++) {
        if (cut[i]) off += 2 * rng.below(2048) + 1;
        ent[i] = Entry{(uint64_t)(uintptr_t)host + rng.below(host_bytes - sizes[i]), (uint64_t)(uintptr_t)dst + off,
                       sizes[i]};
        off += sizes[i];
    }
    std::vector<uint8_t> want(off + 4096, kSentinel);
    for (const Entry& e : ent)
        std::memcpy(&want[e.dst - (uint64_t)(uintptr_t)dst], (const void*)(uintptr_t)e.src, e.size);
    int rc = 0;
    if (path == "direct") {
        CpuPollingThread p(nullptr, nullptr, nullptr, 64u << 20, true, -1);
        if (!p.init_direct_ce()) return 4;
        std::vector<SGEntry> sg(n);
        for (uint32_t i = 0; i < n; i++) sg[i] = SGEntry{ent[i].dst, (const void*)(uintptr_t)ent[i].src, ent[i].size};
        for (int rnd = 0; rnd < rounds && rc == 0; rnd++) {
            std::printf("ragged direct %u entries, %u runs, call %d\n", n, nruns, rnd);
            std::memset(dst, kSentinel, want.size());
            const unsigned zc0 = emu::zero_copy_launches();
            if (p.submit_direct(sg.data(), (int)n) < 0) return 3;
            std::printf("zero-copy launches: %u\n", emu::zero_copy_launches() - zc0);
            rc = check_image(dst, want, "ragged direct", rnd);
        }
    } else {
        auto* q = (DescriptorQueue*)host_alloc(sizeof(DescriptorQueue));
        {
            CpuPollingThread p(q, dst, host, host_bytes, true, -1);
            if (!p.init_copy_engine()) return 4;
            p.start();
            for (int rnd = 0; rnd < rounds && rc == 0; rnd++) {
                std::printf("ragged queue %u entries, %u runs, round %d\n", n, nruns, rnd);
                std::memset(dst, kSentinel, want.size());
                const uint64_t start = q->write_idx;
                Rng lr(seed + (uint64_t)rnd);
                post(q, ent.data(), n, 0, FLAG_LAST_IN_BATCH, lr);
                if (!wait_u64(&q->done_idx, start + n)) {
                    std::printf("ragged queue round %d: done_idx wait timed out\n", rnd);
                    rc = 2;
                    break;
                }
                rc = check_image(dst, want, "ragged queue", rnd);
            }
            p.stop();
        }
        gfd_hip_host_free(q);
    }
    if (rc == 0) std::printf("ragged %s %u runs: pass\n", path.c_str(), nruns);
    gfd_hip_free(dst);
    gfd_hip_host_free(host);
    return rc;
}

// Tiled mode (set_tiled_queue; src/batch_processor.cpp:69-298 of the
// reference), driven as tiled_poller_kernel drives it: one producer per tile
// claims slots chunk by chunk (or the whole tile at once), writes descriptors
// tagged tile << 32 | token with FLAG_LAST_IN_TILE on each chunk's last entry
// and FLAG_LAST_CHUNK_IN_TILE on the tile's last, commits them and waits for
// the tile's cumulative progress word (in HBM or host memory).
int run_tiled(uint32_t tiles, uint32_t T, uint32_t C, uint32_t ts, bool whole, bool dev, int rounds, uint64_t seed) {
    if (tiles == 0 || tiles > (uint32_t)MAX_TILES || C == 0 || T % C != 0 || (uint64_t)tiles * T > QUEUE_SIZE) return 4;
    Rng rng(seed);
    const uint32_t K = T / C;
    const size_t n = (size_t)tiles * T, bytes = n * ts;
    auto* host = (uint8_t*)host_alloc(bytes);
    for (size_t i = 0; i < bytes; i++) host[i] = (uint8_t)rng.next();
    auto* dst = (uint8_t*)dev_alloc(bytes + 4096);
    std::vector<uint8_t> want(bytes + 4096, kSentinel);
    std::memcpy(want.data(), host, bytes);
    auto* tq = (TiledQueue*)host_alloc(sizeof(TiledQueue));
    tq->scheduler.total_tiles = tiles;
    tq->scheduler.tokens_per_tile = T;
    tq->scheduler.tokens_per_chunk = C;
    tq->scheduler.chunks_per_tile = K;
    tq->scheduler.token_size = ts;
    const size_t dev_words = MAX_TILES + TILE_DEVICE_COUNTER_WORDS;
    if (dev) tq->d_tile_chunk_done = (uint64_t*)dev_alloc(dev_words * 8);
    volatile uint64_t* progress = dev ? tq->d_tile_chunk_done : tq->tile_chunk_done;
    int rc = 0;
    {
        CpuPollingThread p(&tq->base, dst, host, bytes, true, -1);
        p.set_tiled_queue(tq);
        if (!p.init_copy_engine()) return 4;
        for (int rnd = 0; rnd < rounds && rc == 0; rnd++) {
            std::printf("tiled %u tiles T=%u C=%u ts=%u whole=%d dev=%d round %d\n", tiles, T, C, ts, (int)whole,
                        (int)dev, rnd);
            p.stop();
            std::memset((void*)&tq->base, 0, sizeof(tq->base));
            std::memset((void*)tq->tile_chunk_done, 0, sizeof(tq->tile_chunk_done));
            if (dev) std::memset(tq->d_tile_chunk_done, 0, dev_words * 8);
            p.reset_stats();
            std::memset(dst, kSentinel, want.size());
            p.start();
            std::atomic<int> timed_out{-1};
            std::vector<std::thread> wg;
            for (uint32_t tile = 0; tile < tiles; tile++)
                wg.emplace_back([&, tile] {
                    Rng lr(seed * 7919u + tile + 131u * (uint64_t)rnd);
                    const uint32_t steps = whole ? 1 : K, per = whole ? T : C;
                    for (uint32_t k = 0; k < steps; k++) {
                        std::vector<Entry> e(per);
                        std::vector<uint32_t> fl(per), tok(per);
                        for (uint32_t i = 0; i < per; i++) {
                            const uint32_t in_tile = k * per + i, g = tile * T + in_tile;
                            e[i] = Entry{(uint64_t)(uintptr_t)host + (uint64_t)g * ts,
                                         (uint64_t)(uintptr_t)dst + (uint64_t)g * ts, ts};
                            fl[i] = (in_tile % C) == C - 1 ? FLAG_LAST_IN_TILE : FLAG_NONE;
                            if (in_tile == T - 1) fl[i] |= FLAG_LAST_CHUNK_IN_TILE;
                            tok[i] = g;
                        }
                        const uint64_t base = __atomic_fetch_add(&tq->base.write_idx, (uint64_t)per, __ATOMIC_RELAXED);
                        for (uint32_t i = 0; i < per; i++) {
                            Descriptor* d = &tq->base.entries[(base + i) % QUEUE_SIZE];
                            d->src_addr = e[i].src;
                            d->dst_addr = e[i].dst;
                            d->size = e[i].size;
                            d->flags = fl[i];
                            d->user_data = ((uint64_t)tile << 32) | tok[i];
                        }
                        uint32_t order[64];
                        for (uint32_t g0 = 0; g0 < per; g0 += 64) {
                            const uint32_t m = std::min<uint32_t>(64, per - g0);
                            for (uint32_t q = 0; q < m; q++) order[q] = q;
                            for (uint32_t q = m; q > 1; q--) std::swap(order[q - 1], order[lr.below(q)]);
                            for (uint32_t q = 0; q < m; q++)
                                __atomic_store_n(&tq->base.entries[(base + g0 + order[q]) % QUEUE_SIZE].sequence,
                                                 base + g0 + order[q] + 1, __ATOMIC_RELEASE);
                        }
                        if (!wait_u64(&progress[tile], (uint64_t)(k + 1) * per)) {
                            timed_out = (int)tile;
                            return;
                        }
                    }
                });
            for (auto& t : wg) t.join();
            if (timed_out >= 0) {
                std::printf("tiled round %d: tile %d wait timed out\n", rnd, timed_out.load());
                rc = 2;
                break;
            }
            rc = check_image(dst, want, "tiled", rnd);
            for (uint32_t tile = 0; tile < tiles && rc == 0; tile++)
                if (progress[tile] != T) {
                    std::printf("tiled round %d: tile %u progress %llu\n", rnd, tile,
                                (unsigned long long)progress[tile]);
                    rc = 3;
                }
        }
        p.stop();
    }
    if (rc == 0) std::printf("tiled: pass\n");
    if (dev) gfd_hip_free(tq->d_tile_chunk_done);
    gfd_hip_host_free(tq);
    gfd_hip_free(dst);
    gfd_hip_host_free(host);
    return rc;
}

// SdmaQueue completion-signal slot reuse.  Copy X (engine 0) depends on copy
// d (engine 1) but sits behind a long copy on its engine; the issuer then
// runs through the whole signal ring so that d's slot comes round again,
// with the new occupant placed on engine 0 behind X.  If the slot were
// reused before X had polled it, X would wait for a copy queued behind
// itself.  Expected: every copy lands and the queue drains.
int run_sdma_slot_reuse() {
    SdmaQueue q;
    if (q.init(0, 2, 1) != 0 || q.num_engines() < 2) return 4;
    const size_t big = 64u << 20, small = 256;
    constexpr int kSlots = 1024;  // SdmaQueue's signal ring
    auto* src = (uint8_t*)host_alloc(big);
    auto* dst = (uint8_t*)dev_alloc(big + (kSlots + 8) * small);
    for (size_t i = 0; i < big; i++) src[i] = (uint8_t)(i * 131 + 7);
    uint8_t* dst_small = dst + big;
    auto small_copy = [&](int ch, uint64_t k, const uint64_t* deps, int nd) {
        return q.copy(ch, (uint64_t)(uintptr_t)(dst_small + k * small), src + (k % 1000) * small, small, nullptr,
                      deps, nd);
    };
    std::printf("sdma slot reuse: ring %d, long copy %zu MiB\n", kSlots, big >> 20);
    int st = small_copy(1, 0, nullptr, 0);                                       // seq 0
    if (!st) st = small_copy(1, 1, nullptr, 0);                                  // seq 1 = d
    if (!st) st = q.copy(0, (uint64_t)(uintptr_t)dst, src, big, nullptr, nullptr, 0);  // seq 2, long
    const uint64_t d = 1;
    if (!st) st = small_copy(0, 3, &d, 1);                                       // seq 3 = X, after d
    for (uint64_t k = 4; !st && k < (uint64_t)kSlots + 1; k++) st = small_copy(1, k, nullptr, 0);
    if (!st) st = small_copy(0, kSlots + 1, nullptr, 0);  // takes d's slot, on X's engine
    if (st) {
        std::printf("sdma slot reuse: copy failed (%d)\n", st);
        return 4;
    }
    if (q.wait_all() != 0) return 3;
    for (size_t i = 0; i < big; i++)
        if (dst[i] != src[i]) {
            std::printf("sdma slot reuse: long copy mismatch at %zu\n", i);
            return 3;
        }
    for (uint64_t k = 0; k <= (uint64_t)kSlots + 1; k++)
        if (k != 2 && std::memcmp(dst_small + k * small, src + (k % 1000) * small, small) != 0) {
            std::printf("sdma slot reuse: copy %llu mismatch\n", (unsigned long long)k);
            return 3;
        }
    std::printf("sdma slot reuse: pass\n");
    gfd_hip_free(dst);
    gfd_hip_host_free(src);
    return 0;
}

}  // namespace

// StagingPool (reference include/gfd/staging_pool.h:50-176 and the pool
// branch of src/cpu_polling.cpp:160-245): the selection rule, acquire /
// release / too small, then Queue pollers that take pool sets while sets are
// free and fit, and allocate their own staging otherwise (a region larger
// than the pool's buffers, or every set taken).  Each poller moves a Queue
// round checked byte for byte; once the pollers are gone every set is free.
int run_staging_pool(int rounds, uint64_t seed) {
    int rc = 0;
    auto expect = [&](bool ok, const char* what) {
        if (!ok && rc == 0) {
            std::printf("staging pool: %s\n", what);
            rc = 3;
        }
    };
    StagingPool& pool = StagingPool::instance();
    expect(!pool.is_initialized() && pool.acquire_buffers(1, -1) == -1, "acquire before init must fail");

    // Selection rule on a table of three sets (buffers are never touched).
    static char dummy[1];
    StagingPool::BufferSet t[3];
    for (auto& b : t) b.bufs[0] = dummy;
    t[0].buf_size = 100, t[0].numa_node = 0;
    t[1].buf_size = 100, t[1].numa_node = 1;
    t[2].buf_size = 50, t[2].numa_node = 1;
    expect(StagingPool::choose_set(t, 3, 100, 1) == 1, "set on the requested node first");
    expect(StagingPool::choose_set(t, 3, 100, 0) == 0, "node 0");
    expect(StagingPool::choose_set(t, 3, 100, -1) == 0, "any node: first free set");
    expect(StagingPool::choose_set(t, 3, 50, 1) == 1, "the first fitting set on the node");
    t[1].in_use = true;
    expect(StagingPool::choose_set(t, 3, 100, 1) == 0, "another node's set when none on the node is free");
    expect(StagingPool::choose_set(t, 3, 60, 1) == 0, "a set too small is skipped");
    expect(StagingPool::choose_set(t, 3, 101, -1) == -1, "nothing fits");

    const uint32_t n = 512, T = 4096;
    const size_t region = (size_t)n * 2 * T;  // the pollers' total_cpu_size
    expect(pool.init(2, region, -1), "init");
    expect(pool.num_sets() == 2, "two sets");
    expect(pool.acquire_buffers(region + 1, -1) == -1, "a request larger than the buffers gets -1");
    const int a = pool.acquire_buffers(region, -1), b = pool.acquire_buffers(region, 0);
    expect(a >= 0 && b >= 0 && a != b, "two sets acquired");
    expect(pool.acquire_buffers(region, -1) == -1, "all sets in use");
    char* bufs[StagingPool::BUFS_PER_SET] = {};
    size_t sz = 0;
    bool hp = true;
    pool.get_buffers(a, bufs, sz, hp);
    expect(sz == region && !hp, "buffer size and hugepage flag");
    for (int i = 0; i < StagingPool::BUFS_PER_SET; i++) {
        expect(bufs[i] != nullptr, "buffer allocated");
        for (int j = 0; j < i; j++) expect(bufs[i] != bufs[j], "distinct buffers");
    }
    pool.release_buffers(a);
    pool.release_buffers(b);
    if (rc) return rc;

    Rng rng(seed);
    auto* host = (uint8_t*)host_alloc(region);
    for (size_t i = 0; i < region; i++) host[i] = (uint8_t)rng.next();
    std::vector<uint32_t> perm(n);
    for (uint32_t i = 0; i < n; i++) perm[i] = i;
    for (uint32_t i = n; i > 1; i--) std::swap(perm[i - 1], perm[rng.below(i)]);
    auto* dst = (uint8_t*)dev_alloc((size_t)n * T);
    std::vector<Entry> ent(n);
    for (uint32_t j = 0; j < n; j++)
        ent[j] = Entry{(uint64_t)(uintptr_t)host + (uint64_t)perm[j] * 2 * T, (uint64_t)(uintptr_t)dst + (uint64_t)j * T, T};
    std::vector<uint8_t> want((size_t)n * T);
    for (uint32_t j = 0; j < n; j++) std::memcpy(&want[(size_t)j * T], (const void*)(uintptr_t)ent[j].src, T);

    // Pollers in creation order: A and B fit the pool and take its two sets,
    // C's region is larger than the pool's buffers, D finds every set taken.
    const size_t totals[4] = {region, region, 2 * region, region};
    const bool pooled[4] = {true, true, false, false};
    std::vector<DescriptorQueue*> qs;
    std::vector<CpuPollingThread*> ps;
    for (int k = 0; k < 4 && rc == 0; k++) {
        qs.push_back((DescriptorQueue*)host_alloc(sizeof(DescriptorQueue)));
        std::memset(qs.back(), 0, sizeof(DescriptorQueue));
        ps.push_back(new CpuPollingThread(qs.back(), dst, host, totals[k], true, -1));
        if (!ps.back()->init_copy_engine()) {
            rc = 4;
            break;
        }
        expect((ps.back()->staging_pool_set() >= 0) == pooled[k], "pool set taken exactly when one fits and is free");
        expect(ps.back()->num_staging_buffers() == 5 && ps.back()->staging_buffer_size() == totals[k],
               "five staging buffers of the poller's region size");
        ps.back()->start();
        for (int rnd = 0; rnd < rounds && rc == 0; rnd++) {
            std::printf("staging pool: poller %d (%s) round %d\n", k, pooled[k] ? "pool set" : "own staging", rnd);
            std::fflush(stdout);
            rc = queue_round(qs.back(), ent, dst, want, seed + (uint64_t)k, rnd, "staging pool");
        }
    }
    for (auto* p : ps) delete p;  // stops each poller and releases its set
    for (auto* q : qs) gfd_hip_host_free(q);
    if (rc == 0) {
        const int x = pool.acquire_buffers(region, -1), y = pool.acquire_buffers(region, -1);
        expect(x >= 0 && y >= 0 && x != y, "both sets free again after the pollers are gone");
        pool.release_buffers(x);
        pool.release_buffers(y);
        pool.shutdown();
        expect(!pool.is_initialized() && pool.acquire_buffers(1, -1) == -1, "shut down");
    }
    gfd_hip_free(dst);
    gfd_hip_host_free(host);
    if (rc == 0) std::printf("staging pool: pass\n");
    return rc;
}

// SdmaQueue::host_source_ok on host memory registered with the runtime: a
// legal SDMA source (and zero-copy kernel source) only when the GPU sees it
// at its host address.
int run_locked_source() {
    int dev = 0;
    SdmaQueue q;
    if (q.init(dev, 2, 1) != 0) return 4;
    std::vector<uint8_t> same(1 << 16), moved(1 << 16);
    emu::note_locked(same.data(), same.size(), (uintptr_t)same.data());
    emu::note_locked(moved.data(), moved.size(), (uintptr_t)moved.data() + (1ull << 40));
    const bool ok_same = q.host_source_ok(same.data() + 100, 4096);
    const bool ok_moved = q.host_source_ok(moved.data() + 100, 4096);
    const bool ok_outside = q.host_source_ok(same.data() + same.size() - 10, 4096);
    emu::note_free(same.data());
    emu::note_free(moved.data());
    if (!ok_same || ok_moved || ok_outside) {
        std::printf("locked source: same-address %d (want 1), other-address %d (want 0), overrun %d (want 0)\n",
                    (int)ok_same, (int)ok_moved, (int)ok_outside);
        return 3;
    }
    std::printf("locked source: pass\n");
    return 0;
}

// submit_direct with the zero-copy worker on: destination-contiguous lists
// with pinned sources (short, long, ragged, one entry, contiguous) become
// worker jobs; a list with pageable sources and one larger than the route's
// limit take the staged route.  Every call's bytes are compared.
int run_worker_direct(uint64_t seed) {
    Rng rng(seed);
    const size_t host_bytes = 24u << 20;
    auto* host = (uint8_t*)host_alloc(host_bytes);
    for (size_t i = 0; i < host_bytes; i += 8) {
        const uint64_t v = rng.next();
        std::memcpy(host + i, &v, 8);
    }
    std::vector<uint8_t> pageable(1u << 20);
    for (auto& b : pageable) b = (uint8_t)rng.next();
    const size_t dst_bytes = 12u << 20;
    auto* dst = (uint8_t*)dev_alloc(dst_bytes);
    struct Case {
        const char* name;
        std::vector<uint32_t> sizes;
        bool pageable, contiguous, want_worker;
    };
    std::vector<Case> cases = {
        {"16 x 4 KiB", std::vector<uint32_t>(16, 4096), false, false, true},
        {"2048 x 512 B", std::vector<uint32_t>(2048, 512), false, false, true},
        {"4 x 256 KiB", std::vector<uint32_t>(4, 256u << 10), false, false, true},
        {"ragged", {}, false, false, true},
        {"one 64 KiB entry", {65536}, false, true, true},
        {"contiguous 32 x 4 KiB", std::vector<uint32_t>(32, 4096), false, true, true},
        {"pageable 64 x 4 KiB", std::vector<uint32_t>(64, 4096), true, false, false},
        {"10 MiB, above the limit", std::vector<uint32_t>(160, 65536), false, false, false},
    };
    for (int i = 0; i < 50; i++) cases[3].sizes.push_back(1 + (uint32_t)rng.below(20000));
    int rc = 0;
    {
        CpuPollingThread p(nullptr, nullptr, nullptr, 16u << 20, true, -1);
        if (!p.init_direct_ce() || p.set_zero_copy_worker(true) != 0) return 4;
        for (const Case& c : cases) {
            if (rc) break;
            std::vector<SGEntry> sg;
            size_t off = 0, src_off = 0;
            for (uint32_t sz : c.sizes) {
                const uint8_t* base = c.pageable ? pageable.data() : host;
                const size_t span = c.pageable ? pageable.size() : host_bytes;
                size_t so = c.contiguous ? src_off : (size_t)rng.below(span - sz);
                if (!c.contiguous && ((sz & 15) == 0)) so &= ~(size_t)15;
                sg.push_back(SGEntry{(uint64_t)(uintptr_t)dst + off, base + so, sz});
                off += sz;
                src_off += sz;
            }
            if (off > dst_bytes) return 4;
            std::vector<uint8_t> want(off + 4096, kSentinel);
            for (const SGEntry& e : sg) std::memcpy(&want[e.dst - (uint64_t)(uintptr_t)dst], e.src, e.size);
            std::memset(dst, kSentinel, want.size());
            const uint64_t jobs0 = p.zero_copy_worker_jobs();
            if (p.submit_direct(sg.data(), (int)sg.size()) < 0) return 3;
            const bool took = p.zero_copy_worker_jobs() == jobs0 + 1;
            std::printf("worker direct %s: %s\n", c.name, took ? "worker" : "other route");
            if (took != c.want_worker) {
                std::printf("worker direct %s: expected the %s route\n", c.name, c.want_worker ? "worker" : "other");
                rc = 3;
            }
            if (rc == 0) rc = check_image(dst, want, c.name, 0);
        }
    }
    gfd_hip_free(dst);
    gfd_hip_host_free(host);
    if (rc == 0) std::printf("worker direct: pass\n");
    return rc;
}

// A pinned source found by one submit_direct call is looked up again by the
// next: between the calls its registration goes away while the addresses stay
// readable to the CPU (a freed pinned buffer whose range a pageable
// allocation now holds).  The second call must not hand those addresses to
// the zero-copy kernel, whose emulation aborts on a source that is not
// pinned, as the GPU faults on one; it takes the staged route instead.
int run_stale_pinned(uint64_t seed) {
    constexpr uint32_t n = 256, t = 4096;  // 1 MiB: the zero-copy route's size
    Rng rng(seed);
    const size_t host_bytes = (size_t)2 * n * t;
    auto* host = (uint8_t*)host_alloc(host_bytes);
    for (size_t i = 0; i < host_bytes; i++) host[i] = (uint8_t)rng.next();
    auto* dst = (uint8_t*)dev_alloc((size_t)n * t);
    std::vector<SGEntry> sg(n);
    std::vector<uint8_t> want((size_t)n * t);
    for (uint32_t i = 0; i < n; i++) {
        const size_t k = (size_t)((i * 37u + 11u) % n);
        sg[i] = SGEntry{(uint64_t)(uintptr_t)dst + (size_t)i * t, host + k * 2 * t, t};
        std::memcpy(&want[(size_t)i * t], host + k * 2 * t, t);
    }
    int rc = 0;
    {
        CpuPollingThread p(nullptr, nullptr, nullptr, 4u << 20, true, -1);
        if (!p.init_direct_ce()) return 4;
        for (int call = 0; call < 3 && rc == 0; call++) {
            if (call == 1) emu::note_free(host);  // registration gone, memory still there
            std::memset(dst, kSentinel, want.size());
            const unsigned zc0 = emu::zero_copy_launches();
            if (p.submit_direct(sg.data(), (int)n) < 0) return 3;
            const unsigned zc = emu::zero_copy_launches() - zc0;
            std::printf("stale pinned: call %d, zero-copy launches %u\n", call, zc);
            if ((call == 0) != (zc == 1)) {
                std::printf("stale pinned: call %d took the %s route\n", call, zc ? "zero-copy" : "staged");
                rc = 3;
            }
            if (rc == 0) rc = check_image(dst, want, "stale pinned", call);
        }
    }
    gfd_hip_free(dst);
    std::free(host);  // its registration was dropped above
    if (rc == 0) std::printf("stale pinned: pass\n");
    return rc;
}

// GatherEngine on its own.  Each round builds a list (uniform tokens, ragged
// sizes, ragged with empty entries, or a long list of small entries that the
// workers scan in parallel), gathers it into one of two staging buffers at a
// random alignment, as a whole-list run (the static split, slices handed over
// in the workers' mailboxes) or a pipelined run whose callback checks each
// chunk as it is reported, and compares every byte and the guard bytes after
// it.  Then the list's source bytes are inverted: a worker copying after
// run() returned would write the inverted bytes, which the check of the same
// image after the next round finds (under ThreadSanitizer that late read is
// also a reported race).  Some rounds pause 3 ms first, past the workers'
// spin limit (GFD_GATHER_SPIN_US), so that jobs also meet sleeping workers.
struct MixChunkCtx {
    const uint8_t* out;
    const uint8_t* want;
    int next;
    bool bad;
};

void mix_check_chunk(void* p, int chunk, size_t off, size_t len) {
    MixChunkCtx* c = (MixChunkCtx*)p;
    if (chunk != c->next || std::memcmp(c->out + off, c->want + off, len) != 0) c->bad = true;
    c->next++;
}

int run_gather_mix(int workers, int rounds, uint64_t seed) {
    Rng rng(seed);
    const size_t src_bytes = 3u << 20, max_total = 1u << 20, guard = 64;
    std::vector<uint8_t> src(src_bytes);
    for (auto& b : src) b = (uint8_t)rng.next();
    std::vector<int> cpus((size_t)workers, -1);
    // On the heap: the engine's 64-byte-aligned members need an aligned
    // object, which ASan's detached stack frames do not guarantee.
    auto engp = std::make_unique<GatherEngine>(cpus);
    GatherEngine& eng = *engp;
    // Room for the image at an offset of up to 2 * guard - 1 and the guard after it.
    std::vector<uint8_t> stg[2] = {std::vector<uint8_t>(max_total + 3 * guard),
                                   std::vector<uint8_t>(max_total + 3 * guard)};
    std::vector<uint8_t> want[2] = {std::vector<uint8_t>(max_total), std::vector<uint8_t>(max_total)};
    size_t want_len[2] = {0, 0}, want_at[2] = {0, 0};
    int whole_runs = 0, chunk_runs = 0, scans = 0;
    for (int r = 0; r < rounds; r++) {
        const int kind = (int)rng.below(4);
        std::vector<SGEntry> e;
        size_t total = 0;
        const uint64_t dst0 = 0x100000 + rng.below(1 << 20);
        auto add = [&](size_t size) {
            const size_t so = rng.below(src_bytes - size + 1);
            e.push_back(SGEntry{dst0 + total, src.data() + so, size});
            total += size;
        };
        if (kind == 0) {  // uniform tokens
            const size_t t = (size_t)64 << rng.below(7);
            const int n = 1 + (int)rng.below((int)std::min<size_t>(700, max_total / t));
            for (int i = 0; i < n; i++) add(t);
        } else if (kind == 1 || kind == 2) {  // ragged, with empty entries in kind 2
            const int n = 1 + (int)rng.below(600);
            for (int i = 0; i < n; i++) add(kind == 2 && rng.below(5) == 0 ? 0 : 1 + rng.below(1500));
        } else {  // long list of small entries: scanned by the workers
            const int n = GatherEngine::kCallerScanMax + 1 + (int)rng.below(3000);
            for (int i = 0; i < n; i++) add(1 + rng.below(120));
        }
        if (total == 0) add(1 + rng.below(100));
        const int b = r & 1;
        const size_t at = guard + rng.below(guard);
        uint8_t* out = stg[b].data() + at;
        std::memset(stg[b].data(), kSentinel, stg[b].size());
        uint8_t* w = want[b].data();
        for (const SGEntry& x : e)
            if (x.size) std::memcpy(w + (x.dst - dst0), x.src, x.size);
        want_len[b] = total;
        want_at[b] = at;
        if (rng.below(8) == 0) std::this_thread::sleep_for(std::chrono::milliseconds(3));
        int uniform_hint = -1;
        if (kind == 0) uniform_hint = (int)rng.below(2);  // 1 (uniform) or 0 (check per entry)
        if (kind == 3 || rng.below(4) == 0) {
            const GatherEngine::ListScan sc = eng.scan(e.data(), (int)e.size());
            scans++;
            if (sc.total != total || !sc.dst_contig) {
                std::fprintf(stderr, "gather mix: round %d scan total %zu (want %zu) dst_contig %d\n", r, sc.total,
                             total, (int)sc.dst_contig);
                return 3;
            }
        }
        if (rng.below(2) == 0) {
            eng.run(e.data(), (int)e.size(), total, (char*)out, 0, nullptr, nullptr, uniform_hint);
            whole_runs++;
        } else {
            eng.set_slice_bytes(4096u << rng.below(4));
            const size_t chunk = 16384u << rng.below(5);
            MixChunkCtx ctx{out, w, 0, false};
            eng.run(e.data(), (int)e.size(), total, (char*)out, chunk, mix_check_chunk, &ctx, uniform_hint);
            chunk_runs++;
            if (ctx.bad) {
                std::fprintf(stderr, "gather mix: round %d a chunk was reported out of order or incomplete\n", r);
                return 3;
            }
        }
        for (int k = 0; k < 2; k++) {  // this round's image, and the previous round's again
            if (k == 1 && r == 0) break;
            const int bb = k == 0 ? b : b ^ 1;
            const uint8_t* o = stg[bb].data() + want_at[bb];
            bool ok = std::memcmp(o, want[bb].data(), want_len[bb]) == 0;
            for (size_t i = 0; i < guard && ok; i++) ok = o[want_len[bb] + i] == kSentinel && o[-(ptrdiff_t)i - 1] == kSentinel;
            if (!ok) {
                std::fprintf(stderr, "gather mix: round %d image of round %d differs (%zu entries, %zu bytes)\n", r,
                             k == 0 ? r : r - 1, e.size(), want_len[bb]);
                return 3;
            }
        }
        for (const SGEntry& x : e)  // the caller may reuse its sources once run() returns
            for (size_t i = 0; i < x.size; i++) ((uint8_t*)x.src)[i] ^= 0xFF;
    }
    std::printf("gather mix: pass (%d whole, %d pipelined, %d scans)\n", whole_runs, chunk_runs, scans);
    return 0;
}

int main(int argc, char** argv) {
    setvbuf(stdout, nullptr, _IOLBF, 0);
    if (argc >= 2 && std::string(argv[1]) == "sdma_slot_reuse") return run_sdma_slot_reuse();
    if (argc >= 2 && std::string(argv[1]) == "locked_source") return run_locked_source();
    if (argc >= 2 && std::string(argv[1]) == "stale_pinned") return run_stale_pinned(7);
    if (argc >= 2 && std::string(argv[1]) == "worker_direct") return run_worker_direct(11);
    if (argc >= 5 && std::string(argv[1]) == "gather_mix")
        return run_gather_mix(std::atoi(argv[2]), std::atoi(argv[3]), std::strtoull(argv[4], nullptr, 0));
    if (argc >= 4 && std::string(argv[1]) == "staging_pool")
        return run_staging_pool(std::atoi(argv[2]), std::strtoull(argv[3], nullptr, 0));
    if (argc >= 10 && std::string(argv[1]) == "tiled")
        return run_tiled((uint32_t)std::atoi(argv[2]), (uint32_t)std::atoi(argv[3]), (uint32_t)std::atoi(argv[4]),
                         (uint32_t)std::atoi(argv[5]), std::atoi(argv[6]) != 0, std::atoi(argv[7]) != 0,
                         std::atoi(argv[8]), std::strtoull(argv[9], nullptr, 0));
    if (argc >= 7 && std::string(argv[1]) == "ragged")
        return run_ragged(argv[2], (uint32_t)std::atoi(argv[3]), (uint32_t)std::atoi(argv[4]), std::atoi(argv[5]),
                          std::strtoull(argv[6], nullptr, 0));
    if (argc >= 5 && std::string(argv[1]) == "sg")
        return run_sg(argv[2], std::atoi(argv[3]), std::strtoull(argv[4], nullptr, 0));
    if (argc >= 7 && std::string(argv[1]) == "queue")
        return run_queue((uint32_t)std::atoi(argv[2]), (uint32_t)std::atoi(argv[3]), std::atoi(argv[4]) != 0,
                         std::atoi(argv[5]), std::strtoull(argv[6], nullptr, 0));
    std::fprintf(stderr,
                 "usage: poller_emu sg <case> <rounds> <seed>\n"
                 "       poller_emu queue <n> <token_bytes> <scattered> <rounds> <seed>\n");
    return 4;
}
