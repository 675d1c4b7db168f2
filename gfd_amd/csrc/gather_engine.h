#pragma once
// GatherEngine: a pool of pinned, spinning worker threads that copy scattered
// host tokens into a contiguous pinned staging buffer with non-temporal
// stores, and report finished chunks in order so the caller can start the
// SDMA copy of each chunk while later chunks are still being gathered.
//
// Role in the reference: CpuPollingThread::parallel_gather +
// gather_worker_loop (src/parallel_gather.cpp:44-116).  The reference splits
// the entries statically into W+1 ranges and joins once; here the
// destination byte range is cut into chunks, chunks into slices, and all
// threads claim slices in order from one atomic counter, so chunk 0 is
// finished by every thread together and its copy can start after a fraction
// of the total gather time.
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <thread>
#include <vector>

#include "gfd/copy_engine.h"

namespace gfd {

// Non-temporal copy: unaligned 64-byte loads, 64-byte-aligned streaming stores,
// memcpy head/tail.  Does not fence; callers fence before publishing.
void stream_copy(void* dst, const void* src, size_t n);
void store_fence();

class GatherEngine {
public:
    // One worker per CPU in worker_cpus (negative id: unpinned).
    explicit GatherEngine(const std::vector<int>& worker_cpus);
    ~GatherEngine();
    GatherEngine(const GatherEngine&) = delete;
    GatherEngine& operator=(const GatherEngine&) = delete;

    int num_workers() const { return (int)threads_.size(); }
    void set_slice_bytes(size_t b) { slice_bytes_ = b < 4096 ? 4096 : b; }
    size_t slice_bytes() const { return slice_bytes_; }
    // Size of the first chunk (0 = chunk_bytes / 8, at least 64 KiB): a short
    // first chunk starts the first copy early.
    void set_first_chunk_bytes(size_t b) { first_chunk_bytes_ = b; }
    // Chunk sizes double from the first chunk up to chunk_bytes (default on).
    void set_chunk_ramp(bool on) { ramp_ = on; }

    // Wake sleeping workers ahead of a job (they spin again until it comes).
    void prewake();

    // Properties of a list the Direct path chooses its route by, computed by
    // the workers and the caller in parallel (a cold 8192-entry list costs
    // the caller alone 10-30 us of DRAM reads).  Lists of up to
    // kCallerScanMax entries are scanned by the caller alone: handing them to
    // the workers costs ~1.8 us, and the zero-copy route reads them again on
    // the caller right after.
    struct ListScan {
        size_t total;
        bool dst_contig, src_contig, uniform;
    };
    ListScan scan(const SGEntry* entries, int count);
    static constexpr int kCallerScanMax = 4096;

    // CLOCK_MONOTONIC ns of the last run() with a chunk callback: entry, after
    // the wait for the previous job's workers, job published, first slice
    // finished (by any thread), and number of threads that copied at least
    // one slice.  Whole-list runs (no callback) leave them as they were.
    struct RunTimes {
        uint64_t entry, idle, built, published, first_slice;
        int copiers, sleepers;
    };
    RunTimes last_run() const { return times_; }

    using ChunkFn = void (*)(void* ctx, int chunk, size_t offset, size_t bytes);

    // Precondition: the entries' destinations are contiguous in order
    // (entry i starts where entry i-1 ends).  Writes entry i's bytes to
    // staging + (entries[i].dst - entries[0].dst).  The destination range
    // [0, total) is cut into chunks (a short first chunk, then chunk_bytes
    // each); on_chunk(ctx, c, off, len) is called on the calling thread, in
    // chunk order, once chunk c's bytes are written and fenced.  Returns as
    // soon as every chunk has been handed to on_chunk.  A null on_chunk (no
    // copy to pipeline) gathers the whole list as one chunk split into
    // num_workers() + 1 equal slices, the reference's static split, and
    // returns once every byte is written and fenced.  Not reentrant: one
    // caller at a time.
    // uniform_hint: 1 = every entry has the same size (slices are placed by
    // division), 0 = not, -1 = check.
    void run(const SGEntry* entries, int count, size_t total, char* staging,
             size_t chunk_bytes, ChunkFn on_chunk, void* ctx, int uniform_hint = -1);

private:
    struct Slice {
        int entry;        // entry holding the slice's first byte
        size_t entry_off; // offset of that byte inside the entry
        size_t off;       // staging offset of the slice
        size_t len;
        int chunk;
    };
    void worker_main(int w, int cpu);
    void do_job(int w);
    void do_slices();
    struct Mailbox;
    void run_whole(const SGEntry* entries, int count, size_t total, char* staging, int uniform_hint);
    static bool take_mailbox_slice(Mailbox& mb, uint32_t job, size_t prefetch_bytes);
    void do_scan_parts();
    void copy_slice(const Slice& s);
    void note_slice(bool& counted);
    Slice slice_at(int s) const;
    int chunk_of(int s) const;

    void publish();
    void wait_workers_out();

    std::vector<std::thread> threads_;
    // Per worker, on a cache line of its own: the job number the caller asks
    // it to join, and whether it is inside a job.  Each line has two users
    // (the caller and that worker), so publishing a job and joining it cost
    // one line transfer per worker, not a queue of them on one shared line.
    //
    // A whole-list job (no chunk callback) also describes the worker's slice
    // in the line: tag is the job the fields belong to (written before go),
    // claimed the last job whose slice someone took, done the last job whose
    // slice is written and fenced.  The worker reads go, finds tag equal to it
    // and claims the slice with one compare-exchange on claimed; the caller
    // can always finish the job alone, taking any slice still unclaimed.  A
    // slice is claimed only while its job is open (claimed older than the
    // job), and the job stays open until that slice is done, so the fields a
    // claimer reads are never rewritten under it.  Such a job touches no
    // other shared job state, so it needs neither open_ nor in_job: workers
    // still leaving an earlier chunked job see none of it change.
    struct alignas(64) Mailbox {
        std::atomic<uint32_t> go{0};
        std::atomic<uint32_t> in_job{0};
        std::atomic<uint32_t> tag{0};
        std::atomic<uint32_t> claimed{0};
        std::atomic<uint32_t> done{0};
        int entry = 0;                     // entry holding the slice's first byte
        const SGEntry* entries = nullptr;  // the list
        char* dst = nullptr;               // staging address of the slice
        size_t entry_off = 0;              // offset of that byte inside the entry
        size_t len = 0;                    // slice bytes
        int count = 0;                     // list entries
    };
    std::unique_ptr<Mailbox[]> mail_;
    // Job counter; 32-bit so idle workers can sleep on it with a futex.
    alignas(64) std::atomic<uint32_t> epoch_{0};
    alignas(64) std::atomic<int> sleepers_{0};
    alignas(64) std::atomic<bool> open_{false};  // job state valid to read
    alignas(64) std::atomic<bool> running_{true};
    alignas(64) std::atomic<int> next_slice_{0};

    // current job (written by the caller before the epoch bump)
    const SGEntry* entries_ = nullptr;
    int count_ = 0;
    char* staging_ = nullptr;
    std::vector<Slice> slices_;  // ragged lists: every slice, precomputed
    int num_slices_ = 0;
    std::vector<size_t> chunk_end_;
    // Uniform lists (every entry esz_ bytes): slices are derived on claim
    // from the chunk table instead of stored.  Rewriting a stored table
    // means writing cache lines every worker read during the previous job,
    // ~16 ns of cross-core invalidation per slice (4 us for 270 slices).
    bool lazy_ = false;
    size_t esz_ = 0;
    std::vector<int> chunk_first_;     // first slice index of each chunk
    std::vector<size_t> chunk_slice_;  // slice length inside each chunk
    std::unique_ptr<std::atomic<int>[]> remaining_;
    int remaining_cap_ = 0;

    // scan job
    struct ScanPart {
        size_t sum;
        bool dst_contig, src_contig, uniform;
        char pad[64 - sizeof(size_t) - 3];
    };
    static constexpr int kScanPartEntries = 512;
    bool scan_job_ = false;  // the open job is a scan
    int scan_parts_ = 0;
    std::vector<ScanPart> scan_out_;
    alignas(64) std::atomic<int> scan_left_{0};

    RunTimes times_{};
    std::atomic<uint64_t> last_prewake_ns_{0};  // prewake() may run on another thread
    std::atomic<uint64_t> first_slice_ns_{0};
    std::atomic<int> copiers_{0};

    // Source bytes of a slice prefetched ahead of the copy (GFD_GATHER_PREFETCH_BYTES;
    // 0 = only the first line of the token four entries ahead).
    size_t prefetch_bytes_ = 6144;
    size_t slice_bytes_ = 128 * 1024;
    size_t first_chunk_bytes_ = 0;
    bool ramp_ = true;
};

}  // namespace gfd
