#pragma once
// CopyEngineManager: asynchronous host-to-HBM copies on the GPU's SDMA
// engines (include/gfd/copy_engine.h:23-98 and src/copy_engine.cpp:13-208
// of the reference, re-designed for ROCm).
//
// Default backend: copies are issued straight to SDMA engines through the HSA
// runtime (one engine per channel when the engines can be pinned), each with
// an HSA completion signal; completion is tracked by sequence number
// ("fences").  Nothing is placed on a GPU compute queue, so copies and
// completion tracking keep running while GPU kernels spin on host-written
// flags.  The HIP-stream backend (GFD_COPY_BACKEND=hip) issues hipMemcpyAsync
// on per-channel non-blocking streams instead.
#include <cstddef>
#include <cstdint>

#include "gfd/hip_shim.h"
#include "gfd/log.h"

namespace gfd {

// 64-bit integer device address (the role CUdeviceptr plays in the
// reference).  It must stay an integer: gathers compute `dst - min_dst`.
using DevicePtr = uint64_t;

// 0 on success, otherwise the HIP / HSA error code.
using Status = int;
constexpr Status GFD_SUCCESS = 0;

#define GFD_HIP_CHECK(call)                                                     \
    do {                                                                        \
        int gfd_err_ = (call);                                                  \
        if (gfd_err_ != 0) {                                                    \
            GFD_LOG_ERROR("HIP error at %s:%d: %s (%d)\n", __FILE__, __LINE__,  \
                          gfd_hip_error_string(gfd_err_), gfd_err_);            \
            return gfd_err_;                                                    \
        }                                                                       \
    } while (0)

// Upper bound on copy channels per manager; DEFAULT_CE_CHANNELS when init()
// is given 0.
constexpr int MAX_CE_CHANNELS = 8;
constexpr int DEFAULT_CE_CHANNELS = 4;

constexpr int MAX_SG_ENTRIES_PER_BATCH = 8192;

// One (dst, src, size) host-to-device request.  Same 24-byte layout as the
// reference SGEntry (include/gfd/copy_engine.h:29-33).
struct SGEntry {
    DevicePtr dst;
    const void* src;
    size_t size;
};
static_assert(sizeof(SGEntry) == 24, "SGEntry must be 24 bytes");

// One destination-contiguous run of a list packed into staging:
// staging [off, off + size) lands at dst.
struct DstRun {
    DevicePtr dst;
    size_t off;
    size_t size;
};

class SdmaQueue;

class CopyEngineManager {
public:
    enum Backend { BACKEND_SDMA = 0, BACKEND_HIP = 1 };

    CopyEngineManager();
    ~CopyEngineManager();
    CopyEngineManager(const CopyEngineManager&) = delete;
    CopyEngineManager& operator=(const CopyEngineManager&) = delete;

    // Set up the channels on `device` (the reference takes a CUcontext; HIP
    // has one primary context per device).  num_channels: 0 = default.
    // The backend comes from GFD_COPY_BACKEND (sdma | hip; default sdma) and
    // engine pinning from GFD_SDMA_PIN (1 default, 0 = runtime's choice).
    Status init(int device, int num_channels = 0);
    void shutdown();

    // Make the manager's device current on the calling thread.  Idempotent;
    // unpin is a no-op kept for API compatibility.
    Status pin_context();
    void unpin_context();

    // Enqueue every entry as an async H2D copy.  count <= channels: one entry
    // per channel round-robin; otherwise each channel takes one contiguous
    // range of entries (src/copy_engine.cpp:103-131).
    Status submit_scatter_gather(const SGEntry* entries, int count);

    // Enqueue one copy on a given channel.
    Status submit_on_channel(int channel, DevicePtr dst, const void* src, size_t size);

    // Enqueue a small copy that starts only after the copies with fence
    // numbers in [after_begin, after_end) have finished, and after copy
    // `also_after` if given (ordered on the copy engines, no host wait).
    // Used for completion flags in HBM.  With one engine per channel
    // (pinned engines, the default) the copy waits for the newest copy of
    // each channel issued since after_begin, at most channels + 1 signals:
    // that covers every copy issued since after_begin, a superset of the
    // range when after_end is not the current fence.
    static constexpr uint64_t kNoFence = ~0ull;
    Status submit_after(DevicePtr dst, const void* src, size_t size, uint64_t after_begin,
                        uint64_t after_end, uint64_t also_after = kNoFence);

    // Fences: every copy gets the next fence number.  fence() is the number the
    // next copy will get; fence_done(f) is true once every copy below f has
    // finished.
    uint64_t fence() const;
    bool fence_done(uint64_t f);
    Status wait_fence(uint64_t f);

    // Block until every copy submitted so far has completed.
    Status wait_completion();
    Status submit_and_wait(const SGEntry* entries, int count);

    // Reference API: record `event` after the most recent copy.  SDMA backend:
    // waits for the copies on the host, after which the event counts as passed.
    Status record_event_on_last_stream(gfd_event_t event);

    // Reference API: make `stream` wait for every outstanding copy.  SDMA
    // backend: waits on the host (the stream then has nothing to wait for).
    Status make_stream_wait_on_all(gfd_stream_t stream);

    uint64_t get_total_submissions() const { return total_submissions_; }
    uint64_t get_total_entries() const { return total_entries_; }
    double get_total_bytes() const { return total_bytes_; }

    bool is_initialized() const { return initialized_; }
    int num_channels() const { return num_channels_; }
    int device() const { return device_; }
    Backend backend() const { return backend_; }
    int num_sdma_engines() const;
    uint32_t sdma_engine_mask() const;
    // True if [p, p + n) is pinned host memory the GPU can read (SDMA backend).
    bool host_source_ok(const void* p, size_t n);
    // Bounds of the pinned allocation the last successful host_source_ok found
    // (both 0 without the SDMA backend).
    void last_pinned_range(uintptr_t* lo, uintptr_t* hi) const;
    // Forget the remembered pinned range (start of each call taking
    // caller-owned sources); mark a range this library allocated pinned and
    // keeps while the manager lives as always legal (staging buffers).
    void forget_pinned_range();
    void trust_range(const void* p, size_t n);

    // Engine timestamps of each copy (SDMA backend only; see SdmaQueue).
    struct CopyTime {
        uint64_t seq, bytes, start_ns, end_ns;
        uint32_t channel, engine;
    };
    void set_copy_timing(bool on);
    size_t read_copy_times(CopyTime* out, size_t max);
    // Now, on the clock of the copy timestamps (0 without the SDMA backend).
    uint64_t copy_clock_ns() const;

private:
    Status issue(int ch, DevicePtr dst, const void* src, size_t size);

    int device_ = 0;
    Backend backend_ = BACKEND_SDMA;
    SdmaQueue* sdma_ = nullptr;
    gfd_stream_t streams_[MAX_CE_CHANNELS] = {};
    gfd_event_t events_[MAX_CE_CHANNELS] = {};
    int num_channels_ = DEFAULT_CE_CHANNELS;
    bool initialized_ = false;
    int next_channel_ = 0;
    int last_channel_ = 0;
    uint32_t dirty_mask_ = 0;
    uint64_t hip_fence_ = 0;

    uint64_t total_submissions_ = 0;
    uint64_t total_entries_ = 0;
    double total_bytes_ = 0;
};

}  // namespace gfd
