// Emulated ZcWorker (gfd_amd/csrc/zc_worker.h) for the host-only build of the
// poller stack: a job's records are copied on the calling thread, each side
// checked to be memory the GPU could reach (pinned host or device memory;
// anything else ends the process, as a GPU page fault would).  The real
// worker is a resident grid on an AQL queue (zc_worker.cpp), which needs a
// GPU.
#include <cstring>

#include "emu.h"
#include "gfd/hip_shim.h"
#include "zc_worker.h"

namespace gfd {

ZcWorker::ZcWorker() = default;

ZcWorker::~ZcWorker() {
    if (table_) gfd_hip_host_free(table_);
}

int ZcWorker::init(int, int workgroups, uint32_t, int capacity) {
    if (workgroups < 1 || capacity < 1) return -1;
    void* p = nullptr;
    if (gfd_hip_host_alloc(&p, (size_t)capacity * sizeof(SGEntry), GFD_HOST_COHERENT) != 0) return -1;
    table_ = static_cast<SGEntry*>(p);
    capacity_ = capacity;
    workgroups_ = workgroups;
    ok_ = true;
    return 0;
}

int ZcWorker::run(int count, uint64_t) {
    if (!ok_ || count < 0 || count > capacity_) return -1;
    if (count == 0) return 0;
    if (!dispatched_) {
        dispatched_ = true;
        launches_++;
    }
    for (int i = 0; i < count; i++) {
        const SGEntry& r = table_[i];
        emu::require_gpu_access(r.src, r.size, "zero-copy worker (source)");
        emu::require_gpu_access((const void*)(uintptr_t)r.dst, r.size, "zero-copy worker (destination)");
        std::memmove((void*)(uintptr_t)r.dst, r.src, r.size);
    }
    jobs_++;
    return 0;
}

}  // namespace gfd
