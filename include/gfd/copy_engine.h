#pragma once
// CopyEngineManager: asynchronous host-to-HBM copies on several SDMA-backed
// HIP streams (include/gfd/copy_engine.h:23-98 and src/copy_engine.cpp:13-208
// of the reference, re-designed for ROCm).
//
// On MI355X a hipMemcpyAsync from pinned host memory to HBM runs on an SDMA
// engine; copies on different streams can run on different engines.  The
// manager owns `num_channels` non-blocking streams (default priority: no
// priority streams are created) and one completion event per stream.
#include <cstddef>
#include <cstdint>

#include "gfd/hip_shim.h"
#include "gfd/log.h"

namespace gfd {

// 64-bit integer device address (the role CUdeviceptr plays in the
// reference).  It must stay an integer: gathers compute `dst - min_dst`.
using DevicePtr = uint64_t;

// 0 on success, otherwise the HIP error code.
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

// Upper bound on copy channels (streams) per manager.  The default used when
// init() is given 0 is DEFAULT_CE_CHANNELS.
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

class CopyEngineManager {
public:
    CopyEngineManager();
    ~CopyEngineManager();
    CopyEngineManager(const CopyEngineManager&) = delete;
    CopyEngineManager& operator=(const CopyEngineManager&) = delete;

    // Create the channel streams and events on `device` (the reference takes a
    // CUcontext; HIP has one primary context per device).
    // num_channels: 0 = DEFAULT_CE_CHANNELS, clamped to MAX_CE_CHANNELS.
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

    // Enqueue one copy on a given channel (used by the pipelined direct path).
    Status submit_on_channel(int channel, DevicePtr dst, const void* src, size_t size);

    // Block until every copy submitted since the last wait has completed.
    Status wait_completion();
    Status submit_and_wait(const SGEntry* entries, int count);

    // Record `event` on the channel used by the most recent submission.
    Status record_event_on_last_stream(gfd_event_t event);

    // Make `stream` wait (on the GPU, not the CPU) for every channel with
    // outstanding copies.
    Status make_stream_wait_on_all(gfd_stream_t stream);

    uint64_t get_total_submissions() const { return total_submissions_; }
    uint64_t get_total_entries() const { return total_entries_; }
    double get_total_bytes() const { return total_bytes_; }

    bool is_initialized() const { return initialized_; }
    int num_channels() const { return num_channels_; }
    int device() const { return device_; }
    gfd_stream_t stream(int ch) const { return streams_[ch]; }

private:
    int device_ = 0;
    gfd_stream_t streams_[MAX_CE_CHANNELS] = {};
    gfd_event_t events_[MAX_CE_CHANNELS] = {};
    int num_channels_ = DEFAULT_CE_CHANNELS;
    bool initialized_ = false;
    int next_channel_ = 0;
    int last_channel_ = 0;
    uint32_t dirty_mask_ = 0;

    uint64_t total_submissions_ = 0;
    uint64_t total_entries_ = 0;
    double total_bytes_ = 0;
};

}  // namespace gfd
