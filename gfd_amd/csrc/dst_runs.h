#pragma once
// Lists whose destinations are not one contiguous range (the reference's
// generic path, src/batch_processor.cpp:14-58,726-831: sort, coalesce, gather
// through staging, one DMA per destination run).
//
// MI355X design: the gather engine always packs a list into staging in list
// order, so no sort is needed.  A list is cut (in list order) into maximal
// destination-contiguous runs; each run occupies one contiguous staging range
// [off, off + size).  While the gather is in flight, every finished chunk of
// staging is copied to the runs it overlaps, one SDMA copy per piece, so the
// copies stay pipelined behind the gather exactly as for a contiguous list.
// Lists with more runs than are worth one copy each take another route (the
// Direct path's zero-copy kernel; the Queue path's per-run copies).
#include <vector>

#include "gfd/copy_engine.h"

namespace gfd {

class CpuPollingThread;

// Up to this many runs a packed gather with one copy per run piece is used.
constexpr int kMaxRunCopies = 64;

// Cut entries[0..count) into destination runs (list order).  Stops once the
// count exceeds max_runs and then returns max_runs + 1; otherwise returns the
// number of runs written to `out`.
inline int dst_runs(const SGEntry* e, int count, int max_runs, std::vector<DstRun>& out) {
    out.clear();
    size_t off = 0;
    for (int i = 0; i < count; i++) {
        if (e[i].size == 0) continue;
        if (!out.empty() && out.back().dst + out.back().size == e[i].dst) {
            out.back().size += e[i].size;
        } else {
            if ((int)out.size() == max_runs) return max_runs + 1;
            out.push_back(DstRun{e[i].dst, off, e[i].size});
        }
        off += e[i].size;
    }
    return (int)out.size();
}

// Gather-engine chunk callback: copy staging [off, off + len) to the runs it
// overlaps.  Chunks arrive in order, so a cursor walks the runs once.
struct RunCopyCtx {
    CpuPollingThread* self;
    CopyEngineManager* ce;
    const char* staging;
    const DstRun* runs;
    int nruns;
    int cursor;
    int channels;
    int next_channel;
    int err;
};

void run_copy_chunk(void* ctx, int chunk, size_t off, size_t len);

}  // namespace gfd
