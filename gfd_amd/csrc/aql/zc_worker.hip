// Persistent zero-copy worker for gfx950: a grid that stays resident on the
// library's own AQL queue and copies scattered (dst, src, size) records
// between pinned host memory and HBM whenever the host rings its doorbell.
// No reference counterpart: it replaces the kernel launch (about 5 us from
// the launch call to the first wave) of the Direct path's zero-copy route for
// short lists, and the copy-engine route of the Queue path's small batches.
//
// Built device-only into a raw code object that the library embeds and
// loads through the HSA runtime (zc_worker.cpp).  A raw AQL dispatch leaves
// the hidden kernel arguments zero, so nothing here reads blockDim / gridDim:
// the workgroup count arrives as an argument and the workgroup size is fixed.
//
// Protocol (host side in zc_worker.cpp):
//   * The host writes a job's records to `table` (pinned memory), then the
//     doorbell word with a release store: bits 0-15 a generation that changes
//     every job, bits 16-39 the record count.  The value ~0 asks the grid to
//     exit.
//   * Wave 0 of workgroup 0 (the leader) polls the doorbell over PCIe, one
//     read in flight at a time.  A new value is published to the other
//     workgroups through HBM (ZcWorkerState::job, an agent-scope release);
//     wave 0 of every other workgroup polls that word with short naps while
//     the workgroup's other waves wait at the workgroup barrier.
//   * Every wave copies its share of the records, releases its stores at
//     system scope and counts itself in ZcWorkerState::waves_done; the last
//     wave resets the count and stores the job's doorbell value to `done`
//     (pinned host memory) with a system-scope release, so every byte is
//     visible to the host once it reads that value.
//   * After idle_ticks (100 MHz wall clock) without a new doorbell value the
//     leader raises ZcWorkerState::exit and the grid ends; the host sees the
//     dispatch's completion signal and dispatches the worker again for its
//     next job.  Records of a job are the units of work: the host cuts large
//     entries of short lists into pieces so that each wave gets one.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gfd/wave_ops.h"

namespace {

constexpr int kWaves = 4;  // per workgroup
constexpr uint64_t kExit = ~0ull;

struct Record {
    uint64_t dst;
    uint64_t src;
    uint64_t size;
};

}  // namespace

// HBM state shared by the grid's workgroups (zc_worker.cpp keeps the same
// layout: 64 bytes).
struct ZcWorkerState {
    uint64_t job;         // the doorbell value the leader published last
    uint32_t waves_done;  // waves finished with the current job
    uint32_t exit;        // 1: every wave leaves
    uint64_t pad[6];
};

// Sets the state a new grid starts from: `last_job` published (already done),
// no wave counted, no exit.  Dispatched ahead of every gfd_zc_worker grid on
// the same queue.
extern "C" __global__ __launch_bounds__(64) void gfd_zc_worker_reset(ZcWorkerState* st, uint64_t last_job) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        st->job = last_job;
        st->waves_done = 0;
        st->exit = 0;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    }
}

extern "C" __global__ __launch_bounds__(kWaves * 64) void gfd_zc_worker(const uint64_t* doorbell, uint64_t* done,
                                                                       const Record* table, ZcWorkerState* st,
                                                                       uint32_t num_blocks, uint64_t last_job,
                                                                       uint64_t idle_ticks) {
    __shared__ gfd::wave::BatchLds lds[kWaves];
    __shared__ uint64_t job_lds;
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint64_t nwaves = (uint64_t)num_blocks * kWaves;
    const uint64_t wave = (uint64_t)blockIdx.x * kWaves + wid;
    uint64_t seen = last_job;
    for (;;) {
        if (wid == 0) {
            uint64_t j = kExit;
            if (blockIdx.x == 0) {
                // The leader: one PCIe read of the doorbell in flight at a time.
                const uint64_t t0 = wall_clock64();
                for (;;) {
                    const uint64_t d = gfd::wave::readlane64(
                        __hip_atomic_load(const_cast<uint64_t*>(doorbell), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM),
                        0);
                    if (d != seen) {
                        j = d;
                        break;
                    }
                    if ((uint64_t)wall_clock64() - t0 > idle_ticks) break;
                }
                if (lane == 0) {
                    if (j == kExit)
                        __hip_atomic_store(&st->exit, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                    else
                        __hip_atomic_store(&st->job, j, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                for (;;) {
                    const uint64_t p = __hip_atomic_load(&st->job, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
                    if (p != seen) {
                        j = p;
                        break;
                    }
                    if (__hip_atomic_load(&st->exit, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT)) break;
                    __builtin_amdgcn_s_sleep(4);
                }
            }
            if (lane == 0) job_lds = j;
        }
        __syncthreads();
        const uint64_t j = job_lds;
        __syncthreads();  // job_lds is written again only after every wave has read it
        if (j == kExit) break;
        seen = j;
        // A launch's dispatch invalidates the caches that may hold pinned host
        // lines; a resident grid must do it per job, or a source the host
        // rewrote since an earlier job could be read stale from L2.  The
        // system-scope acquire does that, and orders the record reads after
        // the doorbell (the host wrote the records first).
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
        const uint64_t count = (j >> 16) & 0xFFFFFFull;
        // Wave w takes records [w * per, ...) strided over the grid, at most
        // 64 at a time; a job of at most nwaves records gives one per wave.
        uint64_t per = (count + nwaves - 1) / nwaves;
        per = per < 1 ? 1 : (per > 64 ? 64 : per);
        const uint64_t stride = nwaves * per;
        for (uint64_t first = wave * per; first < count; first += stride) {
            const uint32_t nb = (uint32_t)(count - first < per ? count - first : per);
            uint64_t md = 0, ms = 0, mn = 0;
            if (lane < nb) {
                const Record r = table[first + lane];
                md = r.dst;
                ms = r.src;
                mn = r.size;
            }
            gfd::wave::copy_batch(16, md, ms, mn, nb, &lds[wid]);
        }
        // System scope: destinations may be pinned host memory as well as HBM.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
        if (lane == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(&st->waves_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            if ((uint64_t)prev + 1 == nwaves) {
                __hip_atomic_store(&st->waves_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(done, j, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    }
}
