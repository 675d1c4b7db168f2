#pragma once
// ZcWorker: a persistent zero-copy copy grid on the library's own AQL queue,
// fed through a doorbell word (device code: aql/zc_worker.hip).  A job is a
// table of (dst, src, size) records in pinned host memory; the worker's 64
// waves copy them (pinned host <-> HBM, in either direction) and signal the
// host through a completion word, so a short copy costs about a PCIe round
// trip plus the data instead of a kernel launch or a copy-engine start.
//
// The queue is created through the HSA runtime, not taken from HIP's pool of
// hardware queues: a kernel that spins on the GPU waiting for this library
// (a Queue-path consumer) can never sit in front of the worker on a shared
// queue.  The grid ends by itself after idle_ms without a job and is
// dispatched again by the next one.
//
// One job at a time: callers hold mutex() while they fill table() and run().
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
    ZcWorker();
    ~ZcWorker();
    ZcWorker(const ZcWorker&) = delete;
    ZcWorker& operator=(const ZcWorker&) = delete;

    // Load the worker for HIP device `device`: code object, AQL queue,
    // completion signal, record table of `capacity` records, state in HBM.
    // workgroups: grid size (4 waves each); idle_ms: idle time after which
    // the grid ends.  Returns 0 or an error.  The grid is dispatched by the
    // first run().
    int init(int device, int workgroups, uint32_t idle_ms, int capacity);
    bool ok() const { return ok_; }

    std::mutex& mutex() { return mu_; }
    // The pinned table the next job copies (capacity() records).
    SGEntry* table() { return table_; }
    int capacity() const { return capacity_; }
    int waves() const { return workgroups_ * 4; }

    // Copy the first `count` records of table() and wait until every byte has
    // landed and is visible to the host and the device.  0, or an error: a
    // dispatch failed, or the job was not done within timeout_us.
    int run(int count, uint64_t timeout_us);

    // Grids dispatched so far (1 + the number of idle exits that a later job
    // followed), and jobs run.
    uint64_t launches() const { return launches_; }
    uint64_t jobs() const { return jobs_; }

private:
    int launch();
    bool grid_finished() const;

    bool ok_ = false;
    std::mutex mu_;
    int workgroups_ = 16;
    uint64_t idle_ticks_ = 0;
    uint64_t gpu_agent_ = 0, cpu_agent_ = 0;
    uint64_t reader_ = 0, executable_ = 0;
    void* queue_ = nullptr;  // hsa_queue_t*
    uint64_t reset_object_ = 0, worker_object_ = 0;
    uint32_t reset_group_ = 0, worker_group_ = 0;
    void* kernarg_ = nullptr;  // kernarg pool memory: reset args, then worker args
    uint64_t signal_ = 0;      // the worker dispatch's completion signal
    uint64_t* words_ = nullptr;  // pinned, coherent: [0] doorbell, [8] done
    SGEntry* table_ = nullptr;
    int capacity_ = 0;
    void* state_ = nullptr;  // HBM: the grid's shared state (64 bytes)
    uint32_t gen_ = 0;
    uint64_t last_done_ = 0;  // doorbell value of the last job the host saw done
    bool dispatched_ = false;
    uint64_t launches_ = 0, jobs_ = 0;
};

}  // namespace gfd
