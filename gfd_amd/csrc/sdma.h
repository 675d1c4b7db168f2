#pragma once
// SdmaQueue: host-to-HBM copies issued straight to the GPU's SDMA engines
// through the HSA runtime (hsa_amd_memory_async_copy[_on_engine]) with one
// HSA completion signal per copy.
//
// Why not HIP streams: a HIP stream's markers and cross-stream waits are AQL
// packets on one of the process's few hardware compute queues.  When a GPU
// kernel spins on a host-written completion flag (queue-mode waits, the
// warp-specialised transfer waves) and a stream of the poller shares that
// hardware queue, the poller's packets sit behind the spinning kernel and
// never run.  SDMA copies with HSA signals never touch a compute queue, and
// the host learns of completion by reading the signals.
//
// Copies get consecutive sequence numbers; retire() advances the completed
// prefix.  Channels map to SDMA engines reported by
// hsa_amd_memory_copy_engine_status (channel i -> i-th available engine), or
// to runtime-chosen engines when engine pinning is off.
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <vector>

namespace gfd {

// The HSA agents (handles) of HIP device `device` and of the host: the GPU
// whose PCI bus id HIP reports for the device, else the device-th GPU agent.
// Returns 0 or an HSA status.
int find_hsa_agents(int device, uint64_t* gpu_agent, uint64_t* cpu_agent);

class SdmaQueue {
public:
    SdmaQueue();
    ~SdmaQueue();
    SdmaQueue(const SdmaQueue&) = delete;
    SdmaQueue& operator=(const SdmaQueue&) = delete;

    // Find the HSA agents of HIP device `device` and the host; set up
    // `channels` channels.  pin_engines: 1 = one SDMA engine per channel,
    // 0 = let the runtime choose.  Returns 0 or an HSA status.
    int init(int device, int channels, int pin_engines);
    bool ok() const { return inited_; }
    int num_channels() const { return channels_; }
    int num_engines() const { return (int)engines_.size(); }
    uint32_t engine_mask() const { return engine_mask_; }

    // Enqueue one host->device copy (or device<-host flag write) on a channel.
    // deps: copies (by sequence number) that must finish first (GPU-side wait).
    // Returns 0 or an HSA status; *seq receives the copy's sequence number.
    int copy(int channel, uint64_t dst, const void* src, size_t bytes, uint64_t* seq = nullptr,
             const uint64_t* deps = nullptr, int ndeps = 0);

    uint64_t issued() const { return next_seq_; }
    // True when every channel is one SDMA engine (its copies finish in the
    // order they were issued on it).
    bool channels_in_order() const { return pin_; }
    // Copies that order everything issued from fence `begin` on, when
    // channels_in_order(): the newest copy of each channel issued at or after
    // `begin` and not yet known complete.  Writes at most max_deps sequence
    // numbers to deps; returns how many, or -1 if there were more.
    int channel_tails(uint64_t begin, uint64_t* deps, int max_deps);
    // Advance past completed copies; returns the first sequence number not yet
    // known complete (every copy below it has finished).
    uint64_t retire();
    bool done(uint64_t seq_end) { return retire() >= seq_end; }
    // Block until every copy with sequence < seq_end has finished.  Returns 0,
    // or -1 if a copy reported an error.
    int wait(uint64_t seq_end);
    int wait_all() { return wait(next_seq_); }
    // Sticky: nonzero once any copy reported failure.
    int error() const { return error_; }

    // Per-copy engine timestamps (hsa_amd_profiling_get_async_copy_time), in
    // ns of the HSA system clock (now_ns()).  Recorded as copies retire while
    // timing is on; read_times drains what has been recorded (any thread).
    // Enabling turns on the runtime's async-copy profiling for the whole
    // process.
    struct CopyTime {
        uint64_t seq, bytes, start_ns, end_ns;
        uint32_t channel, engine;
    };
    void set_timing(bool on);
    size_t read_times(CopyTime* out, size_t max);
    uint64_t now_ns() const;

    // True if [p, p + n) lies in host memory the runtime has pinned and mapped
    // for the GPU (hipHostMalloc / registered), i.e. a legal SDMA source.
    // Pageable memory is not: the caller must copy it another way.
    bool host_source_ok(const void* p, size_t n);
    // Bounds of the pinned allocation the last successful host_source_ok found.
    void last_pinned_range(uintptr_t* lo, uintptr_t* hi) const {
        *lo = ok_lo_;
        *hi = ok_hi_;
    }
    // Forget the remembered pinned range.  Called at the start of every call
    // that takes caller-owned sources: a pinned allocation freed since the
    // last call may have been replaced by pageable memory at the same
    // addresses, which no copy engine or kernel may be handed.
    void forget_pinned_range() { ok_lo_ = ok_hi_ = 0; }
    // A pinned range the owner allocated itself and keeps for as long as this
    // queue lives (staging buffers): a legal source that is never looked up
    // or forgotten.  At most kMaxTrusted ranges; further ones are ignored.
    void trust_range(const void* p, size_t n);

private:
    struct Slot;
    int grow();

    bool inited_ = false;
    bool own_hsa_ = false;
    int channels_ = 0;
    bool pin_ = false;
    uint64_t gpu_agent_ = 0;
    uint64_t cpu_agent_ = 0;
    uint32_t engine_mask_ = 0;
    std::vector<uint32_t> engines_;
    std::vector<uint64_t> signals_;  // ring of hsa_signal_t handles
    // Per ring slot: 1 + the sequence number of the newest copy that waits on
    // the slot's current signal (0 = none).  An engine evaluates a dependency
    // when the dependent copy reaches the head of its ring, by polling the
    // signal's value at that moment, so a slot is not handed to a new copy
    // until every copy that depends on its previous occupant has finished.
    std::vector<uint64_t> waiter_;
    std::vector<uint64_t> ch_last_;  // per channel: 1 + sequence of its newest copy (0 = none)
    uint64_t next_seq_ = 0;
    uint64_t tail_ = 0;  // all seq < tail_ complete
    int error_ = 0;
    uintptr_t ok_lo_ = 0, ok_hi_ = 0;  // last pinned range found
    static constexpr int kMaxTrusted = 8;
    uintptr_t trusted_lo_[kMaxTrusted] = {}, trusted_hi_[kMaxTrusted] = {};
    int ntrusted_ = 0;

    // copy timing
    std::atomic<bool> timing_{false};
    double tick_ns_ = 1.0;
    std::vector<uint64_t> slot_bytes_;
    std::vector<uint32_t> slot_channel_;
    std::mutex times_mu_;
    std::vector<CopyTime> times_;
};

}  // namespace gfd
