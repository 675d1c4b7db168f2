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
// Protocol (host side in zc_worker.cpp).  Host memory is pinned and coherent:
//   * Jobs are numbered 1, 2, ... and posted into a ring of job_slots slots
//     (a power of two).  Slot k holds a header word (one cache line each) and
//     a region of job_cap records.  The host writes job q's records into
//     region q mod job_slots, then its header with a release store:
//     q << 24 | count.  A count of 0xFFFFFF asks the grid to exit.  A slot
//     is reused only after every workgroup has finished the job before.
//   * A record is 32 bytes, two 16-byte halves {dst, size, gen} {src, 0,
//     gen}, gen = the job number's low 24 bits in the last word of each half.
//   * Wave k of workgroup b is slot k * num_blocks + b (consecutive records
//     go to different workgroups, and XCDs).  A job of at most one record per
//     slot gives record s to slot s and stores it at region position b * 8 +
//     k, so that a workgroup's records are 256 contiguous bytes; a larger job
//     is stored in order and gives slot s the run of per = ceil(count /
//     slots) records at s * per (per <= 64: a job holds at most 64 records
//     per slot).
//   * A workgroup is one prefetch wave and kCopyWaves copy waves; copy wave
//     k is slot k * num_blocks + b of workgroup b.  The prefetch wave takes
//     the jobs in order: it polls the header of the next job's ring slot over
//     PCIe (relaxed loads, one read in flight), reads the records of the
//     workgroup's slots (at most 64 each), and
//     stages them in one of two LDS stages, while the copy waves copy the job
//     staged in the other.  For 200 us after a job (a caller that has just
//     copied is likely to copy again) each poll also reads as many of the
//     workgroup's records as its last job had, if that job had at most one
//     record per slot; later polls read the header alone, with short naps.
//     A half read in one request is one snapshot of its cache line, and the
//     host stored the generation after the fields before it, so a half
//     carrying the job's generation holds the job's fields; other halves are
//     read again.  Records read after the header are ordered after it by a
//     system-scope acquire.
//   * Each copy wave copies its records, waits for its stores, and counts
//     itself done in the stage; the last of the kCopyWaves releases the
//     workgroup's stores at agent scope, stores the job number to the
//     workgroup's progress word (pinned host memory, one cache line per
//     workgroup) and frees the stage.  Job q and every job before it are
//     done once every progress word is >= q.
//   * A prefetch wave that finds no new job for idle_ticks (100 MHz wall
//     clock) since its last one stores the dispatch's epoch to the closing
//     word in HBM and stages an exit for its copy waves; every other prefetch
//     wave reads that word in each poll and does the same, so the grid drains
//     within a poll.  The dispatch's
//     completion signal then tells the host, which dispatches the grid again
//     from the first job not done (a job some workgroups had finished is run
//     again in full: copies are idempotent).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gfd/wave_ops.h"

namespace {

constexpr int kCopyWaves = 8;                    // per workgroup, after the prefetch wave
constexpr int kGroupThreads = (kCopyWaves + 1) * 64;
constexpr int kStageRecords = 64;                // per copy wave and job: at most this many records
constexpr uint64_t kExit = ~0ull;     // no job: the grid drains
constexpr uint64_t kExitCount = 0xFFFFFF;  // a header count that asks the grid to exit
constexpr uint64_t kHotTicks = 20000;  // 200 us on the 100 MHz wall clock

// One record: two 16-byte halves, the job's generation in the last word of each.
struct Record {
    uint64_t dst;
    uint32_t size;
    uint32_t gen;
    uint64_t src;
    uint32_t pad;
    uint32_t gen2;
};
static_assert(sizeof(Record) == 32, "record layout");

// One 16-byte half, read as a single system-coherent request (a volatile
// load carries sc0 sc1): no cache line kept from an earlier job can answer it.
__device__ __forceinline__ gfd::wave::vec4u load_half(const char* p) {
    return *reinterpret_cast<const volatile gfd::wave::gvec4u*>((uintptr_t)p);
}

// Per-job device timeline in HBM (zc_worker.cpp reads it): kTraceJobs records
// of 8 words on the 100 MHz wall clock, record (job mod kTraceJobs).  Each
// field is the latest over the grid; a record is reused 64 jobs later with
// larger times, so maxima need no reset:
//   0 a workgroup found the job, 1 a workgroup had the job and its records,
//   3 a workgroup had copied its share, 5 a workgroup had stored its
//   progress word, 6 the job number.
// Word kTraceJobs * 8 after them is the closing word.
constexpr int kTraceJobs = 64;

// flags: kTrace records the timeline (off, no timeline atomic sits on a
// job's path).
constexpr uint32_t kTrace = 1;

__device__ __forceinline__ void trace_max(uint32_t flags, uint64_t* trace, uint64_t job, int field) {
    if (flags & kTrace)
        __hip_atomic_fetch_max(trace + (job & (kTraceJobs - 1)) * 8 + field, (uint64_t)wall_clock64(),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// An LDS stage: one job's header and the records of each copy wave, as the
// two 16-byte halves read from the host.
struct Stage {
    uint64_t job;  // the job staged here, kExit, or 0 (none yet)
    uint64_t header;
    gfd::wave::vec4u rec[kCopyWaves][kStageRecords][2];
};

__device__ __forceinline__ uint64_t lds_load_acquire(uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store_release(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The prefetch wave (wave 0 of a workgroup).
__device__ __forceinline__ void prefetch_wave(const uint64_t* headers, const Record* table, uint64_t* trace,
                                              uint32_t num_blocks, uint32_t flags, uint64_t first_job,
                                              uint64_t idle_ticks, uint64_t epoch, uint32_t job_slots,
                                              uint32_t job_cap, Stage* stage, uint64_t* done_job) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t slots = (uint64_t)num_blocks * kCopyWaves;
    uint64_t* closing = trace + kTraceJobs * 8;
    // Lane l < 2 * kCopyWaves reads half l & 1 of copy wave l / 2's record
    // (slot (l / 2) * num_blocks + blockIdx.x, region position blockIdx.x *
    // kCopyWaves + l / 2) for jobs of at most one record per slot.
    const uint32_t lane_wave = (lane >> 1) & (kCopyWaves - 1);
    const uint64_t lane_slot = (uint64_t)lane_wave * num_blocks + blockIdx.x;
    const uint64_t lane_pos = (uint64_t)blockIdx.x * kCopyWaves + lane_wave;
    uint64_t t_last = wall_clock64();
    uint32_t hot_halves = 0;  // halves the hot polls read: those of the last job's records here
    for (uint64_t q = first_job;; q++) {
        Stage& st = stage[q & 1];
        // The stage last held job q - 2: wait until its copies are done.
        while (lds_load_acquire(&done_job[q & 1]) + 2 < q) __builtin_amdgcn_s_sleep(1);
        const uint64_t ring = q & (job_slots - 1);
        const Record* region = table + ring * job_cap;
        const char* my_half = reinterpret_cast<const char*>(region + lane_pos) + (lane & 1) * 16;
        const uint64_t* header = headers + ring * 8;
        uint64_t h = kExit;
        gfd::wave::vec4u half = {0, 0, 0, 0};
        for (;;) {
            const uint64_t quiet = (uint64_t)wall_clock64() - t_last;
            const bool hot = quiet < kHotTicks;
            const uint64_t c = __hip_atomic_load(closing, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint64_t raw =
                __hip_atomic_load(const_cast<uint64_t*>(header), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (hot && lane < hot_halves) half = load_half(my_half);
            const uint64_t d = gfd::wave::readlane64(raw, 0);
            if ((d >> 24) == q) {
                h = d;
                break;
            }
            if (gfd::wave::readlane64(c, 0) == epoch) break;
            if (quiet > idle_ticks) {
                if (lane == 0) __hip_atomic_store(closing, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if (!hot) __builtin_amdgcn_s_sleep(8);
        }
        const uint64_t count = h & 0xFFFFFFull;
        if (h == kExit || count == kExitCount) {
            if (lane == 0) lds_store_release(&st.job, kExit);
            return;
        }
        if (lane == 0) trace_max(flags, trace, q, 0);
        // A launch's dispatch invalidates the caches that may hold pinned
        // host lines; a resident grid must do it per job, or a source the
        // host rewrote since an earlier job could be read stale.  The
        // workgroup's waves share the CU's L1 and the XCD's L2, so one
        // system-scope acquire here, before the job is staged, does it for
        // the copy waves too.
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
        hot_halves = 0;
        if (count <= slots) {
            // Both halves of each record this workgroup copies must carry the
            // job's generation; stale ones are read again.
            const uint32_t gen = (uint32_t)(q & 0xFFFFFFu);
            const bool want = lane < 2 * kCopyWaves && lane_slot < count;
            for (uint32_t tries = 0; tries < (1u << 20); tries++) {
                const bool stale = want && half[3] != gen;
                if (__ballot(stale) == 0) break;
                half = load_half(my_half);
            }
            if (lane < 2 * kCopyWaves) st.rec[lane_wave][0][lane & 1] = half;
            hot_halves = 2 * (uint32_t)__popcll(__ballot(want) & 0x5555ull);
        } else {
            // Each copy wave's run: per records from position slot * per
            // (per <= kStageRecords: the host posts at most kStageRecords
            // records per slot).  Half i (of 2 * per) of copy wave k is flat
            // index k * 2 * per + i, loaded by lane (index mod 64), eight
            // loads in flight per lane.
            uint64_t per = (count + slots - 1) / slots;
            per = per > kStageRecords ? kStageRecords : per;
            const uint32_t per32 = (uint32_t)per;
            const uint32_t total = kCopyWaves * 2 * per32;  // <= 1024
            for (uint32_t base = 0; base < total; base += 8 * 64) {
                gfd::wave::vec4u v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t idx = base + lane + 64u * u;
                    const uint32_t k = idx / (2 * per32), r = (idx >> 1) - k * per32;
                    uint64_t rec = ((uint64_t)k * num_blocks + blockIdx.x) * per + r;
                    // Branch-free plain loads, all in flight together (a
                    // lane past the run reads record 0, and its value is not
                    // kept; volatile loads would be issued one at a time):
                    // the acquire above has invalidated any line an earlier
                    // job left cached.
                    rec = idx < total && rec < count ? rec : 0;
                    v[u] = gfd::wave::gload((uint64_t)(uintptr_t)(region + rec) + (idx & 1) * 16);
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t idx = base + lane + 64u * u;
                    const uint32_t k = idx / (2 * per32), r = (idx >> 1) - k * per32;
                    const uint64_t rec = ((uint64_t)k * num_blocks + blockIdx.x) * per + r;
                    if (idx < total && rec < count) st.rec[k][r][idx & 1] = v[u];
                }
            }
        }
        if (lane == 0) {
            st.header = h;
            trace_max(flags, trace, q, 1);
            lds_store_release(&st.job, q);
        }
        t_last = wall_clock64();
    }
}

extern "C" __global__ __launch_bounds__(kGroupThreads) void gfd_zc_worker(const uint64_t* headers, uint64_t* progress,
                                                                         const Record* table, uint64_t* trace,
                                                                         uint32_t num_blocks, uint32_t flags,
                                                                         uint64_t first_job, uint64_t idle_ticks,
                                                                         uint64_t epoch, uint32_t job_slots,
                                                                         uint32_t job_cap) {
    __shared__ Stage stage[2];
    __shared__ uint64_t done_job[2];   // stage i: the last job all copy waves finished there
    __shared__ uint32_t done_cnt[2];   // stage i: copy waves done with its current job
    __shared__ gfd::wave::BatchLds lds[kCopyWaves];
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (threadIdx.x == 0) {
        for (int i = 0; i < 2; i++) {
            stage[i].job = 0;
            done_job[i] = first_job - 1;
            done_cnt[i] = 0;
        }
    }
    __syncthreads();
    if (wid == 0) {
        prefetch_wave(headers, table, trace, num_blocks, flags, first_job, idle_ticks, epoch, job_slots, job_cap,
                      stage, done_job);
        return;
    }
    const uint32_t k = wid - 1;  // copy wave index
    const uint64_t slots = (uint64_t)num_blocks * kCopyWaves;
    const uint64_t slot = (uint64_t)k * num_blocks + blockIdx.x;
    for (uint64_t q = first_job;; q++) {
        Stage& st = stage[q & 1];
        uint64_t j;
        while ((j = lds_load_acquire(&st.job)) != q && j != kExit) __builtin_amdgcn_s_sleep(1);
        if (j == kExit) return;
        const uint64_t count = st.header & 0xFFFFFFull;
        if (count <= slots) {
            // At most one record per slot.
            if (slot < count) {
                const gfd::wave::vec4u a = st.rec[k][0][0], b = st.rec[k][0][1];
                uint64_t md = 0, ms = 0, mn = 0;
                if (lane == 0) {
                    md = (uint64_t)a[0] | ((uint64_t)a[1] << 32);
                    mn = (uint64_t)a[2];
                    ms = (uint64_t)b[0] | ((uint64_t)b[1] << 32);
                }
                gfd::wave::copy_batch(16, md, ms, mn, 1, &lds[k]);
            }
        } else {
            // This slot's run of per records, staged (a job holds at most
            // kStageRecords records per slot).
            const uint64_t per = (count + slots - 1) / slots;
            const uint64_t first = slot * per;
            if (first < count) {
                const uint32_t nb = (uint32_t)(count - first < per ? count - first : per);
                uint64_t md = 0, ms = 0, mn = 0;
                if (lane < nb) {
                    const gfd::wave::vec4u a = st.rec[k][lane][0], b = st.rec[k][lane][1];
                    md = (uint64_t)a[0] | ((uint64_t)a[1] << 32);
                    mn = (uint64_t)a[2];
                    ms = (uint64_t)b[0] | ((uint64_t)b[1] << 32);
                }
                gfd::wave::copy_batch(16, md, ms, mn, nb, &lds[k]);
            }
        }
        // This wave's stores have reached the L2 before it counts itself done.
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t prev = 0;
        if (lane == 0)
            prev = __hip_atomic_fetch_add(&done_cnt[q & 1], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
        prev = __builtin_amdgcn_readfirstlane(prev);
        if (prev == kCopyWaves - 1) {
            // The last copy wave of the job here: the workgroup's stores are
            // visible device-wide before its progress word.
            gfd::wave::release_agent();
            if (lane == 0) {
                done_cnt[q & 1] = 0;
                trace_max(flags, trace, q, 3);
                __hip_atomic_store(&progress[(uint64_t)blockIdx.x * 8], q, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
                trace_max(flags, trace, q, 5);
                if (flags & kTrace)
                    __hip_atomic_store(&trace[(q & (kTraceJobs - 1)) * 8 + 6], q, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                lds_store_release(&done_job[q & 1], q);
            }
        }
    }
}
