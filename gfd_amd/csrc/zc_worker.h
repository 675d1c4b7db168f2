#pragma once
// ZcWorker: a persistent zero-copy copy grid on the library's own AQL queue
// (device code: aql/zc_worker.hip).  A job is a list of (dst, src, size)
// records; the host posts it into a ring of kJobSlots job slots in pinned
// host memory, the worker's 64 copy waves ("slots": 8 workgroups of 8 copy
// waves, each workgroup with a prefetch wave that stages the next job's
// records in LDS while the copy waves copy the current one) copy the records
// from pinned host memory into HBM, and each workgroup raises its progress
// word in pinned host memory once it has finished the job.  A short copy thus costs about two PCIe round trips plus the data,
// instead of a kernel launch or a copy-engine start; posting does not wait
// for the copy, so a caller can prepare the next job while one runs, and the
// grid starts it without a round trip through the host.
//
// The queue is created through the HSA runtime, not taken from HIP's pool of
// hardware queues: a kernel that spins on the GPU waiting for this library
// (a Queue-path consumer) can never sit in front of the worker on a shared
// queue.  The grid ends by itself after idle_ms without a job and is
// dispatched again by the next one.
//
// Thread safety: callers hold mutex() (recursive) while they fill table()
// and post() it; post, done, wait and run take it themselves as well.
#include <cstddef>
#include <cstdint>
#include <mutex>

#include "gfd/copy_engine.h"

namespace gfd {

// Cuts a short list of large entries into pieces of at least 4 KiB so that a
// grid of `waves` waves gets about one record per wave; copies the list
// unchanged otherwise (direct_submit.cpp).  *presliced tells which.
int zc_fill_sg_table(const SGEntry* in, int count, size_t total, SGEntry* out, int cap, bool* presliced, int waves);

class ZcWorker {
public:
    static constexpr int kWavesPerGroup = 8;
    static constexpr int kJobSlots = 4;       // jobs that can be posted and not yet done
    static constexpr int kStageRecords = 64;  // records per slot a job may hold
    // Record the device timeline (read_timeline); off, no timeline atomic
    // sits on a job's path.
    static constexpr uint32_t kTrace = 1;

    ZcWorker();
    ~ZcWorker();
    ZcWorker(const ZcWorker&) = delete;
    ZcWorker& operator=(const ZcWorker&) = delete;

    // Load the worker for HIP device `device`: code object, AQL queue,
    // completion signal, kJobSlots job slots of `capacity` records each
    // (between 1 and kStageRecords per slot), the job timeline in HBM.  workgroups: grid
    // size (8 waves each, at most 32 workgroups); idle_ms: idle time after
    // which the grid ends; flags: kTrace or 0.  Returns 0 or an error.  The
    // grid is dispatched by the first post().
    int init(int device, int workgroups, uint32_t idle_ms, int capacity, uint32_t flags = 0);
    bool ok() const { return ok_; }

    std::recursive_mutex& mutex() { return mu_; }
    // The list the next post() copies (capacity() entries, ordinary host memory).
    SGEntry* table() { return list_; }
    int capacity() const { return capacity_; }
    int waves() const { return workgroups_ * kWavesPerGroup; }

    // Post the first `count` entries of table(), or of `list` if given (each
    // at most 4 GiB - 1 bytes, from pinned host memory into device memory),
    // as the next job, after waiting for a free job slot.  Returns the job's
    // number (> 0), or 0: an entry too large, a dispatch failed, or no slot
    // freed within timeout_us (the worker then stays off: ok() is false).
    uint64_t post(int count, uint64_t timeout_us, const SGEntry* list = nullptr);
    // True once job `job` and every job before it have landed and are
    // visible to the device.  Never blocks (it may dispatch the grid again
    // if it has ended).
    bool done(uint64_t job);
    // Wait for done(job); 0, or an error after timeout_us (the worker then
    // stays off).
    int wait(uint64_t job, uint64_t timeout_us);
    // post() and wait(): 0 or an error.
    int run(int count, uint64_t timeout_us);

    // Grids dispatched so far (1 + the number of idle exits that a later job
    // followed), and jobs posted.
    uint64_t launches() const { return launches_; }
    uint64_t jobs() const { return posted_; }

    // Device timeline of the latest jobs (newest first, at most 64), 8 words
    // each on the GPU's 100 MHz wall clock: the last workgroup to find the
    // job, the last to hold it and its records, unused, the last done
    // copying, unused, the last progress word stored, the job number,
    // unused.  Only with kTrace; returns the number of records written to
    // out (8 * max_jobs words).
    int read_timeline(uint64_t* out, int max_jobs);

private:
    int launch();
    bool grid_finished() const;
    // Advance completed_ over the progress words; dispatch the grid again if
    // it has ended with jobs left.  False if a dispatch failed.
    bool poll();
    int wait_until(uint64_t job, uint64_t timeout_us, const char* what);

    bool ok_ = false;
    std::recursive_mutex mu_;
    int workgroups_ = 8;
    uint32_t flags_ = 0;
    uint64_t idle_ticks_ = 0;
    uint64_t gpu_agent_ = 0, cpu_agent_ = 0;
    uint64_t reader_ = 0, executable_ = 0;
    void* queue_ = nullptr;  // hsa_queue_t*
    uint64_t worker_object_ = 0;
    uint32_t worker_group_ = 0;
    void* kernarg_ = nullptr;    // kernarg pool memory: the worker's arguments
    uint64_t signal_ = 0;        // the worker dispatch's completion signal
    uint64_t* words_ = nullptr;  // pinned, coherent: job headers, then the workgroups' progress words
    void* records_ = nullptr;    // pinned, coherent: kJobSlots regions of capacity_ 32-byte records
    SGEntry* list_ = nullptr;    // what callers fill
    int capacity_ = 0;
    uint64_t* trace_ = nullptr;  // HBM: the job timeline, then the closing word
    uint64_t posted_ = 0;        // jobs posted (the last job's number)
    uint64_t completed_ = 0;     // every job up to this one is done
    bool dispatched_ = false;
    uint64_t launches_ = 0;
};

}  // namespace gfd
