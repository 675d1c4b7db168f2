#pragma once
// Wave-specialised scatter-gather framework (HIP sources only).  Same kernel
// interface as the reference's include/gfd/sg_warp_spec.cuh:31-314:
//
//   struct MyCompute { __device__ void operator()(gfd::sg_warp_spec::SGListView v) { ... } };
//   GFD_SG_WARP_SPEC_KERNEL(my_kernel, MyCompute);   // (DescriptorQueue*, SGTaskQueue*, MyCompute)
//
// Wave 0 of each workgroup is the transfer wave, wave 1 the compute wave,
// the last SGDeviceCounters::helpers waves (set by the session per launch)
// transfer helpers; the waves in between return from the loop right after
// its opening barrier, so a kernel may call the loop from every wave and give
// the others work of its own afterwards (a GPU submitter, for instance).
//
// A compute functor that declares `static constexpr bool kSharesLists = true`
// may have several compute waves (waves 1 .. SGDeviceCounters::compute_waves,
// at most SG_MAX_COMPUTE): each landed list then goes to all of them, with
// SGListView::part / parts telling a wave its share, and the list's slot is
// free again once every part is done.  Functors without the declaration see
// each list exactly once, on wave 1, as with the reference.
//
// A functor may instead take the rows of each list one by one, as the
// transfer wave copies them, straight from an LDS ring of SG_ROW_SLOTS rows,
// by declaring `static constexpr bool kStagesRows = true` and
//
//   __device__ uint32_t staged_row_bytes() const;  // R: 1 .. 14 KiB in whole KiB (else: list mode)
//   __device__ void row(const SGRowView& r) const; // must call r.release() once it has read r.data
//
// besides operator() (used when R is not a size the ring takes).  Entries of
// exactly R bytes, 16-byte aligned on both sides, are then loaded by the
// transfer wave, stored to HBM and written into the ring; compute wave c of C
// gets the workgroup's staged rows c, c + C, ... in order.  Other entries are
// copied as usual and not shown to the functor, and lists are still marked
// done once all their bytes have landed.  The rows reach the compute waves
// through LDS instead of being loaded again from HBM, so the compute waves
// put no loads on the vector memory path that the transfer wave's host
// reads take.
//
// The transfer wave claims the next ring index (device-scope atomic on an
// HBM counter), waits for that list to be committed, copies every entry's
// bytes from pinned host memory into HBM itself together with the helpers
// (zero-copy, 16-byte loads over PCIe; the waves claim 64-entry batches of
// the list from an LDS counter, since one wave alone reaches ~3.3 GB/s and a
// CU ~13 GB/s), marks the list done (d_list_done[list_id] in HBM, the header's
// `done` word in host memory) and hands it to the compute wave through one of
// two LDS slots, so the copy of the next list overlaps the compute of this
// one.  The reference routes each list through descriptors and the CPU poller
// instead; the DescriptorQueue argument is kept for the interface and unused.
//
// Lists that a launch's GPU submitters post into the session's HBM queue
// (SGDeviceCounters::dev_ring) are read there: each waiting wave polls its
// own list's header in HBM, and no header or entry crosses PCIe.
//
// Waiting for commits in the host queue: only the wave holding the lowest
// index whose commit no wave has seen (SGDeviceCounters::list_known) reads
// host memory.  When its
// list is committed it reads the next 64 sequences at once (one per lane) and
// advances list_known past the committed run, releasing that many waiting
// waves; the others poll list_known in HBM.  Idle waves thus put one read at
// a time on PCIe instead of one per wave, and a wave whose index is already
// below list_known goes straight to the list's header.
#include <type_traits>

#include "gfd/descriptor_queue.h"
#include "gfd/sg_device_primitives.h"
#include "gfd/sg_task_queue.h"
#include "gfd/wave_ops.h"

namespace gfd {
namespace sg_warp_spec {

// Read-only view of a list whose data is in HBM.
struct SGListView {
    uint32_t list_id;
    uint32_t count;
    uint32_t flags;
    int lane_id;
    uint32_t pool_offset;
    const SGTaskQueue* sq;
    // This wave's share of the list when several compute waves share it
    // (functors with kSharesLists): part in [0, parts).  0 / 1 otherwise.
    uint32_t part;
    uint32_t parts;

    __device__ __forceinline__ DeviceSGEntry get_entry(uint32_t idx) const {
        return sq->entries[(pool_offset + idx) % MAX_SG_POOL_ENTRIES];
    }
    template <typename T>
    __device__ __forceinline__ T* dst_ptr(uint32_t idx) const {
        return reinterpret_cast<T*>(get_entry(idx).dst_addr);
    }
    __device__ __forceinline__ uint32_t entry_size(uint32_t idx) const { return get_entry(idx).size; }
};

struct _SGSlot {
    const SGTaskQueue* ring;  // where the list's entries are
    uint32_t list_id, count, pool_offset, flags;
    int seq;         // k + 1 once the k-th list of this slot is ready
    int free;        // 1 while the slot may be (re)filled
    int parts_done;  // compute waves finished with the slot's current list
};

// At most this many compute waves share a list.
constexpr int SG_MAX_COMPUTE = 3;

template <typename F, typename = void>
struct _shares_lists {
    static constexpr bool value = false;
};
template <typename F>
struct _shares_lists<F, decltype((void)F::kSharesLists)> {
    static constexpr bool value = F::kSharesLists;
};

template <typename F, typename = void>
struct _stages_rows {
    static constexpr bool value = false;
};
template <typename F>
struct _stages_rows<F, decltype((void)F::kStagesRows)> {
    static constexpr bool value = F::kStagesRows;
};

// Staged rows: ring depth and the largest row the ring holds.
constexpr int SG_ROW_SLOTS = 4;
constexpr uint32_t SG_MAX_STAGED_ROW = 14 * 1024;

// One staged row as a compute wave sees it.
struct SGRowView {
    const wave::vec4u* data;  // the row in LDS: this lane's vectors are data[k * 64 + lane_id]
    uint64_t dst;             // where the row landed in HBM
    uint32_t bytes, tag, list_id;
    int lane_id;
    bool first;  // this wave's first row of the launch
    int* slot;
    // Hand the slot back to the transfer wave once data has been read (the
    // workgroup-scope release waits for this wave's LDS reads).
    __device__ __forceinline__ void release() const {
        if (lane_id == 0) __hip_atomic_store(slot, 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
};

struct _SGRowRing {
    wave::vec4u data[SG_ROW_SLOTS][SG_MAX_STAGED_ROW / 16];
    uint64_t dst[SG_ROW_SLOTS];
    uint32_t tag[SG_ROW_SLOTS], list_id[SG_ROW_SLOTS];
    int flag[SG_ROW_SLOTS];  // r + 1 while the slot holds the workgroup's staged row r; 0 once free
};
struct _SGNoRowRing {
    wave::vec4u data[1][1];
    uint64_t dst[1];
    uint32_t tag[1], list_id[1];
    int flag[1];
};

// The functor's staged row size, or 0 for list mode.
template <typename F>
__device__ __forceinline__ uint32_t _staged_row_bytes(const F& f) {
    if constexpr (_stages_rows<F>::value) {
        const uint32_t r = f.staged_row_bytes();
        return (r >= 1024 && r <= SG_MAX_STAGED_ROW && r % 1024 == 0) ? r : 0u;
    } else {
        return 0u;
    }
}

// The idle limit in wall-clock ticks: from the counters in HBM when the
// launch's set-up wrote it there, else from the host queue.
__device__ __forceinline__ uint64_t _idle_limit_ticks(const SGTaskQueue* sq, SGDeviceCounters* cnt) {
    const uint64_t t = __hip_atomic_load(&cnt->idle_ticks, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return t ? t : sg_idle_ticks(wave::load_system32(&sq->idle_limit_ms));
}

// Where ring index idx's header and entries are: the HBM queue of the
// launch's GPU-submitted lists (SGDeviceCounters::dev_ring, from index
// gpu_first on) or the host queue.
__device__ __forceinline__ SGTaskQueue* _ring(SGTaskQueue* sq, SGTaskQueue* dev, uint64_t gpu_first, uint64_t idx) {
    return dev && idx >= gpu_first ? dev : sq;
}

// The waits read the wall clock (s_memrealtime) for their time limits only
// once every kClockPolls polls: the limits are seconds long, so a clock read
// on every poll of every idle wave would buy nothing.
constexpr uint32_t kClockPolls = 64;

// _wait_committed's outcomes.
enum : int { kSgStopped = 0, kSgCommitted = 1, kSgDeadline = 2 };

// Wait until ring index idx is committed: kSgCommitted.  kSgStopped once
// terminate (or the idle limit) ends the wait with nothing committed;
// kSgDeadline once the launch's deadline (0: none) has passed.
__device__ __forceinline__ int _wait_committed(SGTaskQueue* sq, SGDeviceCounters* cnt, uint64_t idx,
                                               uint64_t idle_ticks, uint64_t deadline, SGTaskQueue* dev,
                                               uint64_t gpu_first) {
    const int lane = wave::lane_id();
    const SGList& mine = _ring(sq, dev, gpu_first, idx)->lists[idx % MAX_SG_LISTS];
    const uint64_t t0 = wall_clock64();
    if (dev && idx >= gpu_first) {
        // A GPU-submitted list in HBM: the wave polls its own header there
        // (no host read per poll, so no leader is needed) with relaxed loads
        // (an acquire per poll would invalidate the L2 each time) and one
        // acquire once it is committed; the host queue's terminate is read
        // only every 32nd poll, before the sequence, for the reason given for
        // the leader below.
        for (uint32_t n = 0;; n++) {
            uint32_t term = 0;
            if ((n & 31) == 31) {
                term = __hip_atomic_load(const_cast<uint32_t*>(&sq->terminate), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_SYSTEM);
                if (term) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");  // then the sequence, as below
            }
            if (__hip_atomic_load(const_cast<uint64_t*>(&mine.sequence), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                idx + 1) {
                wave::acquire_agent();  // the header and entries written before the commit
                return kSgCommitted;
            }
            if (term || __hip_atomic_load(&cnt->stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                if (term && lane == 0) __hip_atomic_store(&cnt->stop, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return kSgStopped;
            }
            if ((n & (kClockPolls - 1)) == kClockPolls - 1) {
                if (sg::past(deadline)) return kSgDeadline;
                if (wall_clock64() - t0 > idle_ticks) return kSgStopped;
            }
            __builtin_amdgcn_s_sleep(8);
        }
    }
    for (;;) {
        const uint64_t known = __hip_atomic_load(&cnt->list_known, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (idx < known) {
            // A leader saw this list committed.  The acquire fence pairs with
            // its release when it raised list_known, so the header and
            // entries read next are those written before that commit.
            wave::acquire_agent();
            return kSgCommitted;
        }
        if (idx == known) {
            // Leader.  terminate is read before the sequence.  Whoever sets
            // terminate does so after every list it expects has been
            // committed, with a release store; the acquire (fence) after the
            // load that reads it orders the sequence load after those
            // commits.  So a list still uncommitted once terminate reads 1
            // was never submitted, and the wave can stop at once.  (Read the
            // other way round, a commit could land between the two loads and
            // be dropped.)  Both are polled with relaxed loads and acquired
            // only when they count: an acquire per poll would invalidate the
            // XCD's caches under every other wave there.
            const uint32_t term =
                __hip_atomic_load(const_cast<uint32_t*>(&sq->terminate), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (term) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
            if (__hip_atomic_load(const_cast<uint64_t*>(&mine.sequence), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ==
                idx + 1) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");  // the header and entries written before the commit
                // Find the committed run idx, idx+1, ... and publish it.
                const uint64_t j = idx + (uint64_t)lane;
                const bool c =
                    wave::load_system(&_ring(sq, dev, gpu_first, j)->lists[j % MAX_SG_LISTS].sequence) == j + 1;
                const uint64_t mask = __ballot(c);
                const uint64_t run = (~mask == 0) ? 64 : (uint64_t)__builtin_ctzll(~mask);
                // Release: the 64 sequence loads above (all lanes, one
                // instruction, complete before this store issues) are
                // ordered before the new list_known.
                if (lane == 0)
                    __hip_atomic_fetch_max(&cnt->list_known, idx + (run ? run : 1), __ATOMIC_RELEASE,
                                           __HIP_MEMORY_SCOPE_AGENT);
                return kSgCommitted;
            }
            if (term) {
                if (lane == 0) __hip_atomic_store(&cnt->stop, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return kSgStopped;
            }
            // A GPU submitter that saw every list land raises stop directly.
            if (__hip_atomic_load(&cnt->stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return kSgStopped;
            __builtin_amdgcn_s_sleep(4);
        } else {
            if (__hip_atomic_load(&cnt->stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return kSgStopped;
            // Back off in proportion to how many commits this wave is still
            // waiting for, up to ~3.5 us between polls: device-scope loads
            // bypass the XCD-local L2, so hundreds of idle waves polling at
            // full rate would crowd the fabric the copies use, while a longer
            // nap delays the end of the launch (the waves still waiting then
            // see stop only at their next poll).
            const uint64_t dist = idx - known;
            if (dist < 8) {
                for (uint64_t i = 0; i < dist; i++) __builtin_amdgcn_s_sleep(16);
            } else {
                __builtin_amdgcn_s_sleep(127);
            }
        }
        if (sg::past(deadline)) return kSgDeadline;
        if (wall_clock64() - t0 > idle_ticks) return kSgStopped;
    }
}

// Transfer helpers: up to this many further waves copy batches of the
// transfer wave's current list (SGDeviceCounters::helpers, set per launch).
constexpr int SG_MAX_HELPERS = 3;

// The list the transfer waves copy together.  The leader (wave 0) publishes
// it, leader and helpers claim its 64-entry batches, every helper
// acknowledges it (even with nothing left to claim), and only then does the
// leader publish the next one, so no helper ever reads a job's fields while
// they change.
struct _SGJob {
    const SGTaskQueue* ring;  // where the list's entries are
    uint32_t pool_offset, count;
    int seq;           // k + 1 once the k-th job is published; -1: no more jobs
    int next_batch;    // batches claimed
    int batches_done;  // batches copied
    int acks;          // helpers finished with this job
    unsigned long long bytes;
};

// Claim and copy 64-entry batches of the current job (pool_offset, count);
// adds the batches and bytes copied and returns the job's number of batches.
// The caller passes the job's fields in registers: wave 0 has them from the
// list header, a helper read them after every lane's acquire of job->seq.
// (Lanes 1..63 of wave 0 must not read them back from LDS: lane 0's plain
// stores there are not ordered before other lanes' loads, and the compiler
// does schedule such loads ahead of the stores.)
__device__ __forceinline__ int _sg_copy_batches(_SGJob* job, const SGTaskQueue* sq, uint32_t pool_offset,
                                                uint32_t count, int unroll, wave::BatchLds* lds, int* nbatches_done,
                                                uint64_t* bytes) {
    const int lane = wave::lane_id();
    const int nbatches = (int)((count + wave::kWidth - 1) / wave::kWidth);
    for (;;) {
        int b = 0;
        if (lane == 0) b = __hip_atomic_fetch_add(&job->next_batch, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        b = __builtin_amdgcn_readfirstlane(b);
        if (b >= nbatches) break;
        const uint32_t first = (uint32_t)b * wave::kWidth;
        uint64_t md = 0, ms = 0, mn = 0;
        if (first + lane < count) {
            const DeviceSGEntry e = sq->entries[(pool_offset + first + lane) % MAX_SG_POOL_ENTRIES];
            md = e.dst_addr;
            ms = e.src_addr;
            mn = e.size;
        }
        const uint32_t nb = count - first < (uint32_t)wave::kWidth ? count - first : (uint32_t)wave::kWidth;
        *bytes += wave::copy_batch(unroll, md, ms, mn, nb, lds);
        (*nbatches_done)++;
    }
    return nbatches;
}

// Transfer wave, staged rows of V KiB: copy the list's entries, staging each
// row of exactly V KiB (16-byte aligned) into the next ring slot once its
// compute wave has freed it; other entries are copied as they are.  Adds the
// bytes copied; false if a slot was never freed (the compute waves stalled).
template <int V>
__device__ __forceinline__ bool _sg_stage_rows(const SGTaskQueue* ring, uint32_t pool_offset, uint32_t count,
                                               uint32_t list_id, _SGRowRing* rr, int* nrows, uint64_t* bytes) {
    using wave::vec4u;
    constexpr uint32_t kRow = (uint32_t)V * 1024;
    const int lane = wave::lane_id();
    for (uint32_t first = 0; first < count; first += wave::kWidth) {
        uint64_t md = 0, ms = 0, mn = 0;
        uint32_t tag = 0;
        if (first + lane < count) {
            const DeviceSGEntry e = ring->entries[(pool_offset + first + lane) % MAX_SG_POOL_ENTRIES];
            md = e.dst_addr;
            ms = e.src_addr;
            mn = e.size;
            tag = e.tag;
        }
        const bool st = mn == kRow && ((md | ms) & 15) == 0;
        // Other entries (rare beside the rows: a skipped row has size 0)
        // are copied one by one with a light loop, which keeps the kernel's
        // registers within what the row's V vectors leave.
        for (uint64_t other = __ballot(mn != 0 && !st); other; other &= other - 1) {
            const int j = __builtin_ctzll(other);
            const uint64_t n = wave::readlane64(mn, j);
            wave::copy<4>(wave::readlane64(md, j), wave::readlane64(ms, j), n);
            *bytes += n;
        }
        for (uint64_t rows = __ballot(st); rows; rows &= rows - 1) {
            const int j = __builtin_ctzll(rows);
            const uint64_t s0 = wave::readlane64(ms, j), d0 = wave::readlane64(md, j);
            const uint32_t tj = (uint32_t)__builtin_amdgcn_readlane((int)tag, j);
            const int r = *nrows;
            const int slot = r % SG_ROW_SLOTS;
            if (!wave::wait_lds_eq(&rr->flag[slot], 0)) return false;
            vec4u v[V];
#pragma unroll
            for (int k = 0; k < V; k++) v[k] = wave::gload(s0 + (uint64_t)(k * wave::kWidth + lane) * 16);
#pragma unroll
            for (int k = 0; k < V; k++) wave::gstore(d0 + (uint64_t)(k * wave::kWidth + lane) * 16, v[k]);
#pragma unroll
            for (int k = 0; k < V; k++) rr->data[slot][k * wave::kWidth + lane] = v[k];
            if (lane == 0) {
                rr->dst[slot] = d0;
                rr->tag[slot] = tj;
                rr->list_id[slot] = list_id;
                wave::lds_store(&rr->flag[slot], r + 1);  // release: the row and its fields first
            }
            *nrows = r + 1;
            *bytes += kRow;
        }
    }
    return true;
}

// (Instantiated only for functors that stage rows.)
template <bool kOn>
__device__ __forceinline__ bool _sg_stage_rows_kb(uint32_t kb, const SGTaskQueue* ring, uint32_t pool_offset,
                                                  uint32_t count, uint32_t list_id, _SGRowRing* rr, int* nrows,
                                                  uint64_t* bytes) {
    if constexpr (!kOn) {
        return false;
    } else {
        switch (kb) {
#define GFD_SG_STAGE_CASE(n) \
    case n: return _sg_stage_rows<n>(ring, pool_offset, count, list_id, rr, nrows, bytes);
            GFD_SG_STAGE_CASE(1) GFD_SG_STAGE_CASE(2) GFD_SG_STAGE_CASE(3) GFD_SG_STAGE_CASE(4) GFD_SG_STAGE_CASE(5)
            GFD_SG_STAGE_CASE(6) GFD_SG_STAGE_CASE(7) GFD_SG_STAGE_CASE(8) GFD_SG_STAGE_CASE(9) GFD_SG_STAGE_CASE(10)
            GFD_SG_STAGE_CASE(11) GFD_SG_STAGE_CASE(12) GFD_SG_STAGE_CASE(13) GFD_SG_STAGE_CASE(14)
#undef GFD_SG_STAGE_CASE
            default: return false;
        }
    }
}

// cnt_arg: the launch's counters (sg_device_counters(sq)) when the kernel
// was given their address; otherwise each wave finds them through the host
// queue, one read across PCIe as it starts.
template <typename ComputeFn>
__device__ __forceinline__ void _sg_transfer_warp_loop(DescriptorQueue* dq, SGTaskQueue* sq, ComputeFn compute_fn,
                                                       SGDeviceCounters* cnt_arg = nullptr) {
    (void)dq;
    __shared__ _SGSlot slots[2];
    __shared__ int terminated;
    __shared__ _SGJob job;
    __shared__ wave::BatchLds batch_lds[1 + SG_MAX_HELPERS];  // per transfer wave
    constexpr bool kStaging = _stages_rows<ComputeFn>::value;
    __shared__ typename std::conditional<kStaging, _SGRowRing, _SGNoRowRing>::type rr;
    // Staged-row mode (kStagesRows functors with a row size the ring takes).
    const uint32_t staged_bytes = _staged_row_bytes(compute_fn);
    const bool staged = staged_bytes != 0;
    const int w = wave::wave_id();
    const int lane = wave::lane_id();
    if (threadIdx.x < 2) {
        slots[threadIdx.x].seq = 0;
        slots[threadIdx.x].free = 1;
        slots[threadIdx.x].parts_done = 0;
    }
    if (threadIdx.x == 0) {
        terminated = 0;
        job.seq = 0;
    }
    if (kStaging && threadIdx.x < SG_ROW_SLOTS) rr.flag[threadIdx.x] = 0;
    __syncthreads();

    SGDeviceCounters* const cnt = cnt_arg ? cnt_arg : sg_device_counters(sq);
    const int nwaves = (int)(blockDim.x / wave::kWidth);
    const bool has_compute = nwaves > 1;
    // Helpers are the last `helpers` waves of the workgroup (never wave 0 or 1).
    int helpers = (int)__hip_atomic_load(&cnt->helpers, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (helpers > SG_MAX_HELPERS) helpers = SG_MAX_HELPERS;
    if (helpers > nwaves - 2) helpers = nwaves > 2 ? nwaves - 2 : 0;
    if (staged) helpers = 0;  // the leader stages rows itself; helper waves return at once
    const int first_helper = nwaves - helpers;
    const int unroll = wave::transfer_unroll(gridDim.x * (1u + (unsigned)helpers));
    // Compute waves 1 .. ncompute (never into the helpers).
    int ncompute = 1;
    if (_shares_lists<ComputeFn>::value || staged) {
        ncompute = (int)__hip_atomic_load(&cnt->compute_waves, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ncompute > SG_MAX_COMPUTE) ncompute = SG_MAX_COMPUTE;
        if (ncompute > first_helper - 1) ncompute = first_helper - 1;
        if (ncompute < 1) ncompute = 1;
    }

    if (w == 0) {
        // ---------------- transfer wave (leader)
        const uint64_t idle_ticks = _idle_limit_ticks(sq, cnt);
        const uint64_t deadline = sg::launch_deadline(cnt);
        // Timeline of this launch's lists, when the session asks for one.
        const uint64_t t_start = (uint64_t)wall_clock64();
        SGTraceList* const trace =
            reinterpret_cast<SGTraceList*>(__hip_atomic_load(&cnt->trace, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        const uint64_t trace_cap = __hip_atomic_load(&cnt->trace_cap, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t list_base = __hip_atomic_load(&cnt->list_base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        SGTaskQueue* const dev =
            reinterpret_cast<SGTaskQueue*>(__hip_atomic_load(&cnt->dev_ring, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        const uint64_t gpu_first =
            list_base + __hip_atomic_load(&cnt->host_lists, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint64_t nlists = 0;
        int nrows = 0;  // rows staged (staged-row mode)
        for (uint64_t iter = 0;; iter++) {
            const int s = (int)(iter & 1);
            if (has_compute && !staged && !wave::wait_lds_eq(&slots[s].free, 1)) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, SG_ERR_SLOT_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            const uint64_t t_claimed = (uint64_t)wall_clock64();
            uint64_t idx = 0;
            if (lane == 0) idx = sg::atomic_add_dev(&cnt->list_claim, 1);
            idx = wave::broadcast0(idx);
            const int got = _wait_committed(sq, cnt, idx, idle_ticks, deadline, dev, gpu_first);
            if (got != kSgCommitted) {
                if (got == kSgDeadline && lane == 0)
                    __hip_atomic_fetch_or(&cnt->error, SG_ERR_DEADLINE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            SGTaskQueue* const ring = _ring(sq, dev, gpu_first, idx);
            SGList& l = ring->lists[idx % MAX_SG_LISTS];
            const uint32_t pool_offset = l.pool_offset, count = l.count, list_id = l.list_id, flags = l.flags;
            if (lane == 0) wave::store_system(&l.sequence, 0);  // claimed
            const uint64_t t_ready = (uint64_t)wall_clock64();

            uint64_t bytes = 0;
            if (staged) {
                if (!_sg_stage_rows_kb<kStaging>(staged_bytes / 1024, ring, pool_offset, count, list_id,
                                                 reinterpret_cast<_SGRowRing*>(&rr), &nrows, &bytes)) {
                    if (lane == 0)
                        __hip_atomic_fetch_or(&cnt->error, SG_ERR_SLOT_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                wave::acquire_agent();
                wave::release_agent();  // the list's bytes are visible device-wide
            } else {
            // Publish the copy job, copy batches with the helpers, wait for
            // every batch and every helper's acknowledgement.
            if (lane == 0) {
                job.ring = ring;
                job.pool_offset = pool_offset;
                job.count = count;
                job.next_batch = 0;
                job.batches_done = 0;
                job.acks = 0;
                job.bytes = 0;
                wave::lds_store(&job.seq, (int)iter + 1);
            }
            int mine = 0;
            const int nbatches =
                _sg_copy_batches(&job, ring, pool_offset, count, unroll, &batch_lds[0], &mine, &bytes);
            if (lane == 0) {
                __hip_atomic_fetch_add(&job.bytes, (unsigned long long)bytes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                wave::lds_add(&job.batches_done, mine);
            }
            if (helpers > 0 &&
                (!wave::wait_lds_eq(&job.batches_done, nbatches) || !wave::wait_lds_eq(&job.acks, helpers))) {
                if (lane == 0) __hip_atomic_fetch_or(&cnt->error, SG_ERR_HELPER_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            bytes = __hip_atomic_load(&job.bytes, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
            wave::acquire_agent();
            wave::release_agent();  // the list's bytes (all transfer waves') are visible device-wide
            }
            nlists++;
            if (lane == 0) {
                if (trace && idx - list_base < trace_cap)
                    trace[idx - list_base] = SGTraceList{t_claimed, t_ready, (uint64_t)wall_clock64(), blockIdx.x, list_id};
                if (list_id < (uint32_t)MAX_SG_LISTS)
                    __hip_atomic_store(&sg_list_done_words(cnt)[list_id], 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                sg::atomic_add_dev(&cnt->entries_done, count);
                sg::atomic_add_dev(&cnt->bytes_done, bytes);
                const uint64_t landed =
                    __hip_atomic_fetch_add(&cnt->lists_done, 1ull, __ATOMIC_SEQ_CST, __HIP_MEMORY_SCOPE_AGENT) + 1;
                wave::store_system(&l.done, idx + 1);
                // Host code and host submitters read the marker in the host queue.
                if (ring != sq) wave::store_system(&sq->lists[idx % MAX_SG_LISTS].done, idx + 1);
                // The launch's last list (sg_stop_when_landed): end the launch.
                const uint64_t stop_at = __hip_atomic_load(&cnt->stop_at, __ATOMIC_SEQ_CST, __HIP_MEMORY_SCOPE_AGENT);
                if (stop_at != 0 && landed >= stop_at) {
                    __hip_atomic_store(const_cast<uint32_t*>(&sq->terminate), 1u, __ATOMIC_RELEASE,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
                    __hip_atomic_store(&cnt->stop, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (has_compute && !staged) {
                    slots[s].ring = ring;
                    slots[s].list_id = list_id;
                    slots[s].count = count;
                    slots[s].pool_offset = pool_offset;
                    slots[s].flags = flags;
                    slots[s].free = 0;
                    wave::lds_store(&slots[s].seq, (int)(iter / 2) + 1);
                }
            }
        }
        if (lane == 0) {
            wave::lds_store(&job.seq, -1);  // helpers exit
            wave::lds_store(&terminated, 1);
            if (trace && blockIdx.x < __hip_atomic_load(&cnt->trace_blocks, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                reinterpret_cast<SGTraceBlock*>(trace + trace_cap)[blockIdx.x] =
                    SGTraceBlock{t_start, (uint64_t)wall_clock64(), nlists,
                                 ((uint64_t)(uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) |
                                     (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4)};
        }
    } else if (helpers > 0 && w >= first_helper) {
        // ---------------- transfer helper: copies batches of the leader's
        // jobs; bounded like the compute wave.
        const uint64_t limit = _idle_limit_ticks(sq, cnt) + 100000000ull;
        const uint64_t deadline = sg::launch_deadline(cnt);
        for (int want = 1;;) {
            int seq = 0;
            const uint64_t t0 = wall_clock64();
            for (uint32_t n = 1;; n++) {
                seq = wave::lds_load(&job.seq);
                if (seq < 0 || seq >= want) break;
                // The leader publishes -1 when it stops, deadline included;
                // a second past it means the leader itself is stuck.
                if ((n & (kClockPolls - 1)) == 0 &&
                    (wall_clock64() - t0 > limit || (deadline && sg::past(deadline + 100000000ull)))) {
                    if (lane == 0) __hip_atomic_fetch_or(&cnt->error, SG_ERR_HELPER_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    seq = -1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            if (seq < 0) break;
            int mine = 0;
            uint64_t bytes = 0;
            _sg_copy_batches(&job, job.ring, job.pool_offset, job.count, unroll, &batch_lds[1 + w - first_helper],
                             &mine, &bytes);
            wave::release_agent();  // this wave's stores are visible device-wide before it reports
            if (lane == 0) {
                __hip_atomic_fetch_add(&job.bytes, (unsigned long long)bytes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                wave::lds_add(&job.batches_done, mine);
                wave::lds_add(&job.acks, 1);
            }
            want = seq + 1;
        }
    } else if (has_compute && staged && w >= 1 && w <= ncompute) {
        // ---------------- compute wave(s), staged rows: wave w takes the
        // workgroup's staged rows w - 1, w - 1 + ncompute, ...; bounded like
        // the list-mode compute wave below.
        if constexpr (kStaging) {
            const uint64_t limit = _idle_limit_ticks(sq, cnt) + 100000000ull;
            const uint64_t deadline = sg::launch_deadline(cnt);
            bool first = true;
            for (int i = w - 1;; i += ncompute) {
                const int s = i % SG_ROW_SLOTS;
                bool ready = false;
                const uint64_t t0 = wall_clock64();
                for (uint32_t n = 1;; n++) {
                    if (wave::lds_load(&rr.flag[s]) == i + 1) {
                        ready = true;
                        break;
                    }
                    if (wave::lds_load(&terminated)) {  // every row is staged by now: row i is here or never comes
                        ready = wave::lds_load(&rr.flag[s]) == i + 1;
                        break;
                    }
                    if ((n & (kClockPolls - 1)) == 0 &&
                        (wall_clock64() - t0 > limit || (deadline && sg::past(deadline + 100000000ull)))) {
                        if (lane == 0)
                            __hip_atomic_fetch_or(&cnt->error, SG_ERR_COMPUTE_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                if (!ready) break;
                SGRowView view;
                view.data = rr.data[s];
                view.dst = rr.dst[s];
                view.bytes = staged_bytes;
                view.tag = rr.tag[s];
                view.list_id = rr.list_id[s];
                view.lane_id = lane;
                view.first = first;
                view.slot = &rr.flag[s];
                compute_fn.row(view);
                first = false;
            }
        }
    } else if (has_compute && w >= 1 && w <= ncompute) {
        // ---------------- compute wave(s): bounded by the transfer wave's
        // idle limit (plus 1 s), the longest the transfer wave can stay silent.
        const uint64_t limit = _idle_limit_ticks(sq, cnt) + 100000000ull;
        const uint64_t deadline = sg::launch_deadline(cnt);
        for (uint64_t k = 0;; k++) {
            const int s = (int)(k & 1);
            const int want = (int)(k / 2) + 1;
            bool ready = false;
            const uint64_t t0 = wall_clock64();
            for (uint32_t n = 1;; n++) {
                if (wave::lds_load(&slots[s].seq) == want) {
                    ready = true;
                    break;
                }
                if (wave::lds_load(&terminated)) {
                    ready = wave::lds_load(&slots[s].seq) == want;
                    break;
                }
                if ((n & (kClockPolls - 1)) == 0 &&
                    (wall_clock64() - t0 > limit || (deadline && sg::past(deadline + 100000000ull)))) {
                    if (lane == 0) __hip_atomic_fetch_or(&cnt->error, SG_ERR_COMPUTE_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            if (!ready) break;
            wave::acquire_agent();
            SGListView view;
            view.list_id = slots[s].list_id;
            view.count = slots[s].count;
            view.flags = slots[s].flags;
            view.lane_id = lane;
            view.pool_offset = slots[s].pool_offset;
            // Uniform across the wave: kept in scalar registers.
            view.sq = reinterpret_cast<const SGTaskQueue*>(
                wave::readlane64((uint64_t)(uintptr_t)slots[s].ring, 0));
            view.part = (uint32_t)(w - 1);
            view.parts = (uint32_t)ncompute;
            compute_fn(view);
            if (lane == 0) {
                // The last part frees the slot.  Its reset of parts_done is
                // ordered before the slot's next list by the release of free
                // (the transfer wave acquires free before refilling the slot,
                // and the compute waves acquire seq before their next add).
                const int done = ncompute == 1 ? 1
                                               : __hip_atomic_fetch_add(&slots[s].parts_done, 1, __ATOMIC_ACQ_REL,
                                                                        __HIP_MEMORY_SCOPE_WORKGROUP) + 1;
                if (done == ncompute) {
                    if (ncompute > 1)
                        __hip_atomic_store(&slots[s].parts_done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    wave::lds_store(&slots[s].free, 1);
                }
            }
        }
    }
    // further waves return to the caller
}

// Largest workgroup of an SG kernel: 1 transfer + up to 3 compute + up to
// 3 helper waves fit in 8 waves (two per SIMD, 256 registers each).
constexpr int SG_MAX_BLOCK = 512;

}  // namespace sg_warp_spec
}  // namespace gfd

// Kernel generation macro (block = 64 * (1 + compute + helper waves) threads).
#define GFD_SG_WARP_SPEC_KERNEL(kernel_name, ComputeFnType)                                 \
    __global__ __launch_bounds__(gfd::sg_warp_spec::SG_MAX_BLOCK) void kernel_name(         \
        gfd::DescriptorQueue* dq, gfd::SGTaskQueue* sq, ComputeFnType compute_fn) {         \
        gfd::sg_warp_spec::_sg_transfer_warp_loop(dq, sq, compute_fn);                      \
    }
