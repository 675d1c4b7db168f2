// Emulated ZcWorker (gfd_amd/csrc/zc_worker.h) for the host-only build of the
// poller stack.  post() keeps the job in its ring slot and returns at once;
// the copies happen later, one job per done() call (every job up to the one
// waited for in wait()), so a caller that publishes completion before done()
// says so finds its destination unwritten.  Each side of a record is checked
// to be memory the GPU could reach (pinned host or device memory; anything
// else ends the process, as a GPU page fault would).  The real worker is a
// resident grid on an AQL queue (zc_worker.cpp), which needs a GPU.
#include <cstring>

#include "emu.h"
#include "gfd/hip_shim.h"
#include "zc_worker.h"

namespace gfd {

// records_ holds kJobSlots rings slots of capacity_ entries; trace_ (no
// timeline here) holds each ring slot's entry count.
ZcWorker::ZcWorker() = default;

ZcWorker::~ZcWorker() {
    delete[] list_;
    delete[] static_cast<SGEntry*>(records_);
    delete[] reinterpret_cast<int*>(trace_);
}

int ZcWorker::init(int, int workgroups, uint32_t, int capacity, uint32_t flags) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (workgroups < 1 || workgroups > 32 || capacity < workgroups * kWavesPerGroup ||
        capacity > workgroups * kWavesPerGroup * kStageRecords)
        return -1;
    list_ = new SGEntry[capacity];
    records_ = new SGEntry[(size_t)kJobSlots * capacity];
    trace_ = reinterpret_cast<uint64_t*>(new int[kJobSlots]);  // per ring slot: the job's count
    capacity_ = capacity;
    workgroups_ = workgroups;
    flags_ = flags;
    ok_ = true;
    return 0;
}

// Run the oldest job not yet run.
bool ZcWorker::poll() {
    if (completed_ >= posted_) return true;
    const uint64_t job = completed_ + 1;
    const int ring = (int)(job & (kJobSlots - 1));
    const int count = reinterpret_cast<int*>(trace_)[ring];
    const SGEntry* e = static_cast<SGEntry*>(records_) + (size_t)ring * capacity_;
    for (int i = 0; i < count; i++) {
        emu::require_gpu_access(e[i].src, e[i].size, "zero-copy worker (source)");
        emu::require_gpu_access((const void*)(uintptr_t)e[i].dst, e[i].size, "zero-copy worker (destination)");
        std::memmove((void*)(uintptr_t)e[i].dst, e[i].src, e[i].size);
    }
    completed_ = job;
    return true;
}

bool ZcWorker::done(uint64_t job) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (completed_ < job) poll();
    return completed_ >= job;
}

int ZcWorker::wait_until(uint64_t job, uint64_t, const char*) {
    while (completed_ < job && completed_ < posted_) poll();
    return completed_ >= job ? 0 : -1;
}

int ZcWorker::wait(uint64_t job, uint64_t timeout_us) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    return wait_until(job, timeout_us, "a job");
}

uint64_t ZcWorker::post(int count, uint64_t timeout_us, const SGEntry* list) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (!ok_ || count <= 0 || count > capacity_) return 0;
    const SGEntry* in = list ? list : list_;
    for (int i = 0; i < count; i++)
        if (in[i].size > 0xFFFFFFFFull) return 0;
    const uint64_t job = posted_ + 1;
    if (job > (uint64_t)kJobSlots && wait_until(job - kJobSlots, timeout_us, "a free job slot") != 0) return 0;
    if (!dispatched_) {
        dispatched_ = true;
        launches_++;
    }
    const int ring = (int)(job & (kJobSlots - 1));
    std::memcpy(static_cast<SGEntry*>(records_) + (size_t)ring * capacity_, in, (size_t)count * sizeof(SGEntry));
    reinterpret_cast<int*>(trace_)[ring] = count;
    posted_ = job;
    return job;
}

int ZcWorker::run(int count, uint64_t timeout_us) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (count == 0) return ok_ ? 0 : -1;
    const uint64_t job = post(count, timeout_us);
    return job ? wait(job, timeout_us) : -1;
}

int ZcWorker::read_timeline(uint64_t*, int) { return 0; }

}  // namespace gfd
