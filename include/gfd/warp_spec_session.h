#pragma once
// Session managers for the wave-specialised frameworks (the reference's
// include/gfd/warp_spec_session.h:14-258 and src/*_session.cpp: the same class
// names, configuration fields and lifecycle: construct, launch(kernel, fn),
// synchronize(), reset(), get_stats()).
//
// MI355X design: the kernels move the data themselves (zero-copy loads from
// pinned host memory, see include/gfd/warp_spec.h and sg_warp_spec.h), so a
// session's launches need no CPU poller.  get_poller() still returns a live
// CpuPollingThread owned by the session, created on first use over the
// session's own descriptor ring (WarpSpecSession: tiled mode over its
// TiledQueue; SGWarpSpecSession: queue mode over its DescriptorQueue).  Its
// start()/stop() bracket a kernel the caller launches itself, its stats
// count what the session's transfer waves landed as well as what it copied
// itself, and after a caller-launched SG kernel its stop() leaves the session
// ready for the next launch.  launch() is a template defined for HIP
// translation units.
#include <chrono>
#include <cstdint>
#include <deque>
#include <functional>
#include <vector>

#include "gfd/cpu_polling.h"
#include "gfd/hip_shim.h"
#include "gfd/sg_task_queue.h"
#include "gfd/tiled_queue.h"

namespace gfd {

// Transfer helper waves per workgroup when the configuration leaves the count
// to the session (negative): about 32 transfer waves per launch, at most 3
// helpers.  Measured on MI355X: one wave moves ~3.3 GB/s and one CU ~13 GB/s
// over PCIe, and 32 waves with 16 loads in flight each fill the link, so
// small grids (1-8 workgroups) gain up to ~1.6x from helpers while large ones
// gain nothing.
inline int auto_helper_waves(int grid) {
    if (grid <= 0) grid = 1;
    const int h = (32 + grid - 1) / grid - 1;
    return h < 0 ? 0 : (h > 3 ? 3 : h);
}

struct WarpSpecConfig {
    // required
    uint32_t total_tokens = 0;
    uint32_t token_size = 0;
    void* cpu_src = nullptr;   // pinned host memory
    void* gpu_dst = nullptr;   // HBM

    // optional
    uint32_t tokens_per_tile = 128;
    uint32_t tokens_per_chunk = 0;  // 0 = automatic
    int num_blocks = 0;             // 0 = one workgroup per tile, at most one per CU
    int numa_node = 0;              // kept for API compatibility
    bool use_copy_engine = true;    // kept for API compatibility (data moves zero-copy)
    bool double_buffer = false;
    bool per_tile_mode = false;     // one chunk per tile
    // Transfer helper waves per workgroup (an addition to the reference's API): they copy
    // pieces of each tile next to the transfer wave, so one workgroup keeps up
    // to 4x the loads in flight.  Negative: auto_helper_waves(grid), set by
    // the session.  Fewer if the workgroup would pass 1024 threads.
    int transfer_helper_waves = -1;

    // Chunk size: about 64 KiB (tokens <= 512 B), 128 KiB, or 256 KiB (tokens
    // >= 64 KiB) per chunk, a power of two, at least 4 tokens, and at most 8
    // chunks per tile (4 with double buffering, so a workgroup stays within
    // 1024 threads with 64-lane waves) — the reference's heuristic with the
    // wave64 limit (include/gfd/warp_spec_session.h:33-52).
    uint32_t effective_tokens_per_chunk() const {
        if (per_tile_mode) return tokens_per_tile;
        if (tokens_per_chunk > 0) return tokens_per_chunk;
        uint64_t target = 128 * 1024;
        if (token_size <= 512) target = 64 * 1024;
        else if (token_size >= 65536) target = 256 * 1024;
        uint32_t c = token_size ? (uint32_t)(target / token_size) : 1;
        if (c < 4) c = 4;
        if (c > tokens_per_tile) c = tokens_per_tile;
        const uint32_t max_k = double_buffer ? 4 : 8;
        const uint32_t min_c = tokens_per_tile / max_k;
        if (min_c > 0 && c < min_c) c = min_c;
        uint32_t p = 1;
        while (p * 2 <= c) p *= 2;
        return p;
    }
    uint32_t total_tiles() const { return tokens_per_tile ? total_tokens / tokens_per_tile : 0; }
    uint32_t chunks_per_tile() const { return tokens_per_tile / effective_tokens_per_chunk(); }
    int helper_waves() const {
        const int k = (int)chunks_per_tile();
        const int room = 16 - (double_buffer ? 1 + 2 * k : 1 + k);
        const int h = transfer_helper_waves > 0 ? transfer_helper_waves : 0;
        return h < room ? h : (room > 0 ? room : 0);
    }
    // 1 transfer wave + K (or 2K) compute waves + helper waves, 64 lanes each.
    int block_size() const {
        const int k = (int)chunks_per_tile();
        return (double_buffer ? 1 + 2 * k : 1 + k) * 64 + helper_waves() * 64;
    }
};

class WarpSpecSession {
public:
    explicit WarpSpecSession(const WarpSpecConfig& config);
    ~WarpSpecSession();
    WarpSpecSession(const WarpSpecSession&) = delete;
    WarpSpecSession& operator=(const WarpSpecSession&) = delete;

    // Launch a GFD_WARP_SPEC_KERNEL(_DB) kernel: (TiledQueue*, gpu_dst, cpu_src, fn).
    template <typename KernelFn, typename ComputeFn>
    void launch(KernelFn kernel, ComputeFn compute_fn, gfd_stream_t stream = nullptr);

    struct LaunchParams {
        TiledQueue* tq;
        void* gpu_buffer;
        const void* cpu_base;
        unsigned grid;
        unsigned block;
    };
    LaunchParams get_launch_params() const;

    // Wait for the launch to finish.  False if the kernel reported a stalled
    // hand-off or the stream returned an error.
    bool synchronize();
    // Clear tile progress and the tile counter for another launch.
    void reset();

    struct Stats {
        uint64_t descriptors_processed;  // tokens landed
        uint64_t bytes_transferred;
        double elapsed_ms;
        double bandwidth_gbps;
    };
    Stats get_stats() const;

    TiledQueue* get_queue() const { return tq_; }
    // The session's poller (created on first call; nullptr if the session
    // failed to construct).  reset() clears its stats, as the reference's does.
    CpuPollingThread* get_poller() const;
    // The configuration in effect (helper waves resolved).
    const WarpSpecConfig& config() const { return config_; }
    bool ok() const { return ok_; }
    uint64_t error_bits() const { return error_bits_; }
    uint64_t tiles_done() const { return tiles_done_; }

    // Internal: called by launch().
    void before_launch(gfd_stream_t stream);

private:
    WarpSpecConfig config_;
    TiledQueue* tq_ = nullptr;
    uint64_t* d_signals_ = nullptr;  // MAX_TILES progress words + TileDeviceCounters
    int num_blocks_ = 0;
    bool ok_ = false;
    bool running_ = false;  // launched, not yet synchronized
    gfd_stream_t stream_ = nullptr;
    uint64_t error_bits_ = 0;
    uint64_t tiles_done_ = 0;
    std::chrono::steady_clock::time_point launch_time_;
    double last_elapsed_ms_ = 0;
    void* trace_buf_ = nullptr;  // HBM: trace_cap_ SGTraceList + num_blocks_ SGTraceBlock
    uint32_t trace_cap_ = 0;
    mutable CpuPollingThread* poller_ = nullptr;
    // Tiles landed by this session's launches since reset(): a poller created
    // later starts from them.
    uint64_t landed_tiles_total_ = 0;
};

struct SGWarpSpecConfig {
    int num_compute_warps = 0;  // compute waves per workgroup (0 -> 1, as in the reference)
    int num_blocks = 0;         // 0 = min(CU count, 64)
    int numa_node = 0;          // kept for API compatibility
    bool use_copy_engine = true;
    int max_lists = MAX_SG_LISTS;
    int max_entries = MAX_SG_POOL_ENTRIES;
    uint32_t idle_limit_ms = 0;  // transfer waves give up after this long without a list (0 = 30 s)
    // Transfer helper waves per workgroup (an addition to the reference's API, 0..3): they
    // copy 64-entry batches of each list next to the transfer wave.
    // Negative: auto_helper_waves(grid), set by the session.
    int transfer_helper_waves = -1;

    int block_size() const {
        const int h = transfer_helper_waves > 0 ? transfer_helper_waves : 0;
        return (1 + (num_compute_warps > 0 ? num_compute_warps : 1) + h) * 64;
    }
};

class SGWarpSpecSession {
public:
    explicit SGWarpSpecSession(const SGWarpSpecConfig& config);
    ~SGWarpSpecSession();
    SGWarpSpecSession(const SGWarpSpecSession&) = delete;
    SGWarpSpecSession& operator=(const SGWarpSpecSession&) = delete;

    // Host submission: entries into the pool, header, release fence, commit.
    // Blocks while the ring or the pool is full of lists not yet landed.
    // Returns the list's ring index, or ~0 on a timeout / invalid argument.
    uint64_t submit_sg_list(const DeviceSGEntry* entries, uint32_t count, uint32_t list_id,
                            uint32_t flags = SG_FLAG_HOST_SUBMITTED);

    SGTaskQueue* get_sg_queue() const { return sq_; }
    DescriptorQueue* get_desc_queue() const { return dq_; }
    // The session's poller (created on first call; nullptr if the session
    // failed to construct).  For a kernel the caller launches itself
    // (test/test_sg_gpu_submit.cu's flow: launch, get_poller()->start(),
    // device synchronize, get_poller()->stop()), stop() reads back what the
    // launch landed (get_stats(), the poller's stats) and prepares the
    // session's counters for the next launch.  Such a kernel starts on the
    // state a new session, reset(), that stop(), or synchronize() once the
    // poller exists, leave: no helper waves, one compute wave, no deadline.
    CpuPollingThread* get_poller() const;

    // Launch a GFD_SG_WARP_SPEC_KERNEL kernel: (DescriptorQueue*, SGTaskQueue*, fn).
    template <typename KernelFn, typename ComputeFn>
    void launch(KernelFn kernel, ComputeFn compute_fn, gfd_stream_t stream = nullptr);

    // Wait until every host-submitted list (plus `extra_gpu_lists` lists
    // submitted by GPU waves during the launch) has landed, then terminate the
    // transfer waves and wait for the kernel.  False on timeout or error.
    bool synchronize(uint64_t extra_gpu_lists = 0);
    void reset();

    struct Stats {
        uint64_t descriptors_processed;  // entries landed
        uint64_t bytes_transferred;
        double elapsed_ms;
        double bandwidth_gbps;
    };
    Stats get_stats() const;

    bool ok() const { return ok_; }
    bool running() const { return running_; }  // launched and not yet synchronized
    uint64_t error_bits() const { return error_bits_; }
    uint64_t lists_landed() const { return lists_done_; }  // during the last launch
    int num_blocks() const { return num_blocks_; }
    int helper_waves() const { return config_.transfer_helper_waves; }
    int block_size() const { return config_.block_size(); }

    // Internal: called by launch().  helper_waves < 0: the configured count;
    // kernels whose extra waves have other work (a GPU submitter) pass their own.
    // compute_waves < 0: num_compute_warps (used only by functors that share
    // lists between compute waves).  deadline_ms > 0: every wait of the
    // launch gives up that long after it starts (launches whose lists all
    // come from GPU submitters; see SGDeviceCounters::deadline).
    void before_launch(gfd_stream_t stream, int helper_waves = -1, int compute_waves = -1,
                       uint32_t deadline_ms = 0, SGTaskQueue* gpu_ring = nullptr);
    // An SGTaskQueue in HBM for GPU-submitted lists (allocated on first call;
    // nullptr if that fails).  A launch whose GPU submitters post there
    // passes it to before_launch as gpu_ring (SGDeviceCounters::dev_ring).
    SGTaskQueue* device_ring();
    // The idle limit in effect (idle_limit_ms, 0 meaning 30 s), which GPU
    // submitter launches also take as their deadline.
    uint32_t idle_limit_ms() const { return config_.idle_limit_ms ? config_.idle_limit_ms : 30000u; }
    int compute_waves() const { return config_.num_compute_warps > 0 ? config_.num_compute_warps : 1; }
    // True when GPU submitters posting at most `lists` lists and `entries`
    // entries in the next launch can never find the ring, a ring slot or the
    // entry pool still in use (the host's queued lists included), so they
    // may skip those waits.
    bool gpu_lists_fit(uint64_t lists, uint64_t entries) const;

    // Per-list device timeline (not in the reference).  From the next launch
    // on, the transfer waves record each of the launch's first max_lists
    // lists (SGTraceList, in ring order) and each workgroup (SGTraceBlock);
    // 0 switches it off.  False if the record buffer cannot be allocated.
    bool enable_trace(uint32_t max_lists);
    // The last launch's records (after synchronize()); false if tracing is off.
    bool read_trace(std::vector<SGTraceList>& lists, std::vector<SGTraceBlock>& blocks) const;

private:
    struct Pending {
        uint64_t idx;
        uint64_t pool_begin;
        uint32_t count;
    };
    bool list_done(uint64_t idx) const;
    void retire_done();
    bool wait_until(const std::function<bool()>& cond, double limit_ms);
    double wait_limit_ms() const;
    // Take in a finished launch's device counters: stats, consumed ring and
    // pool positions, error bits, the poller's stats.
    void absorb(const SGDeviceCounters& c);
    // Device counters for a kernel the caller launches itself, written with
    // blocking copies.
    void prepare_raw_launch();
    // The poller's stop hook: a caller-launched kernel has finished.
    void after_raw_launch();

    SGWarpSpecConfig config_;
    SGTaskQueue* sq_ = nullptr;
    SGTaskQueue* dev_ring_ = nullptr;  // HBM: lists posted by GPU submitters
    DescriptorQueue* dq_ = nullptr;
    int num_blocks_ = 0;
    bool ok_ = false;
    bool running_ = false;
    gfd_stream_t stream_ = nullptr;
    uint64_t consumed_lists_ = 0;    // ring index where the next launch's claims start
    uint64_t consumed_entries_ = 0;  // pool index every consumed list lies below
    std::deque<Pending> pending_;    // host-submitted lists not yet seen landed, in order
    uint64_t error_bits_ = 0;
    uint64_t entries_done_ = 0, bytes_done_ = 0, lists_done_ = 0;  // last launch
    std::chrono::steady_clock::time_point launch_time_;
    double last_elapsed_ms_ = 0;
    void* trace_buf_ = nullptr;  // HBM: trace_cap_ SGTraceList + num_blocks_ SGTraceBlock
    uint32_t trace_cap_ = 0;
    mutable CpuPollingThread* poller_ = nullptr;
    // Landed since reset(), so a poller created later starts from them.
    uint64_t landed_entries_total_ = 0, landed_bytes_total_ = 0, landed_lists_total_ = 0;
};

// The spelling SgWarpSpecSession, which callers also use for this class.
using SgWarpSpecSession = SGWarpSpecSession;

}  // namespace gfd

#ifdef __HIPCC__
#include <hip/hip_runtime.h>

template <typename KernelFn, typename ComputeFn>
void gfd::WarpSpecSession::launch(KernelFn kernel, ComputeFn compute_fn, gfd_stream_t stream) {
    before_launch(stream);
    const LaunchParams p = get_launch_params();
    hipLaunchKernelGGL(kernel, dim3(p.grid), dim3(p.block), 0, (hipStream_t)stream, p.tq, p.gpu_buffer, p.cpu_base,
                       compute_fn);
}

template <typename KernelFn, typename ComputeFn>
void gfd::SGWarpSpecSession::launch(KernelFn kernel, ComputeFn compute_fn, gfd_stream_t stream) {
    before_launch(stream);
    hipLaunchKernelGGL(kernel, dim3(num_blocks_), dim3(config_.block_size()), 0, (hipStream_t)stream, dq_, sq_,
                       compute_fn);
}
#endif
