// CopyEngineManager over HIP streams (declaration: include/gfd/copy_engine.h).
// Behaviour follows src/copy_engine.cpp:13-208 of the reference: per-channel
// completion events, round-robin for few entries and one contiguous range of
// entries per channel otherwise, dirty-mask waits.
#include "gfd/copy_engine.h"

namespace gfd {

CopyEngineManager::CopyEngineManager() = default;

CopyEngineManager::~CopyEngineManager() { shutdown(); }

Status CopyEngineManager::init(int device, int num_channels) {
    if (initialized_) return GFD_SUCCESS;
    device_ = device;
    num_channels_ = num_channels > 0 ? num_channels : DEFAULT_CE_CHANNELS;
    if (num_channels_ > MAX_CE_CHANNELS) num_channels_ = MAX_CE_CHANNELS;
    GFD_HIP_CHECK(gfd_hip_set_device(device_));
    for (int i = 0; i < num_channels_; i++) {
        GFD_HIP_CHECK(gfd_hip_stream_create(&streams_[i]));
        GFD_HIP_CHECK(gfd_hip_event_create(&events_[i], 0));
    }
    next_channel_ = 0;
    last_channel_ = 0;
    dirty_mask_ = 0;
    initialized_ = true;
    GFD_LOG_DEBUG("copy engine: %d channels on device %d\n", num_channels_, device_);
    return GFD_SUCCESS;
}

void CopyEngineManager::shutdown() {
    if (!initialized_) return;
    gfd_hip_set_device(device_);
    for (int i = 0; i < num_channels_; i++) {
        if (streams_[i]) {
            gfd_hip_stream_synchronize(streams_[i]);
            gfd_hip_stream_destroy(streams_[i]);
            streams_[i] = nullptr;
        }
        if (events_[i]) {
            gfd_hip_event_destroy(events_[i]);
            events_[i] = nullptr;
        }
    }
    initialized_ = false;
}

Status CopyEngineManager::pin_context() {
    if (!initialized_) return GFD_SUCCESS;
    GFD_HIP_CHECK(gfd_hip_set_device(device_));
    return GFD_SUCCESS;
}

void CopyEngineManager::unpin_context() {}

Status CopyEngineManager::submit_on_channel(int ch, DevicePtr dst, const void* src, size_t size) {
    if (!initialized_) return GFD_SUCCESS;
    ch %= num_channels_;
    GFD_HIP_CHECK(gfd_hip_memcpy_h2d_async(dst, src, size, streams_[ch]));
    GFD_HIP_CHECK(gfd_hip_event_record(events_[ch], streams_[ch]));
    dirty_mask_ |= 1u << ch;
    last_channel_ = ch;
    total_bytes_ += (double)size;
    total_submissions_++;
    total_entries_++;
    return GFD_SUCCESS;
}

Status CopyEngineManager::submit_scatter_gather(const SGEntry* entries, int count) {
    if (!initialized_ || count <= 0) return GFD_SUCCESS;
    uint32_t used = 0;
    if (count <= num_channels_) {
        for (int i = 0; i < count; i++) {
            int ch = next_channel_;
            next_channel_ = (next_channel_ + 1) % num_channels_;
            GFD_HIP_CHECK(gfd_hip_memcpy_h2d_async(entries[i].dst, entries[i].src,
                                                   entries[i].size, streams_[ch]));
            used |= 1u << ch;
            last_channel_ = ch;
            total_bytes_ += (double)entries[i].size;
        }
    } else {
        int per = (count + num_channels_ - 1) / num_channels_;
        for (int ch = 0; ch < num_channels_; ch++) {
            int b = ch * per;
            if (b >= count) break;
            int e = b + per < count ? b + per : count;
            for (int i = b; i < e; i++) {
                GFD_HIP_CHECK(gfd_hip_memcpy_h2d_async(entries[i].dst, entries[i].src,
                                                       entries[i].size, streams_[ch]));
                total_bytes_ += (double)entries[i].size;
            }
            used |= 1u << ch;
            last_channel_ = ch;
        }
        next_channel_ = 0;
    }
    for (uint32_t m = used; m; m &= m - 1) {
        int ch = __builtin_ctz(m);
        GFD_HIP_CHECK(gfd_hip_event_record(events_[ch], streams_[ch]));
    }
    dirty_mask_ |= used;
    total_submissions_++;
    total_entries_ += (uint64_t)count;
    return GFD_SUCCESS;
}

Status CopyEngineManager::wait_completion() {
    if (!initialized_ || dirty_mask_ == 0) return GFD_SUCCESS;
    for (uint32_t m = dirty_mask_; m; m &= m - 1) {
        int ch = __builtin_ctz(m);
        GFD_HIP_CHECK(gfd_hip_event_synchronize(events_[ch]));
    }
    dirty_mask_ = 0;
    return GFD_SUCCESS;
}

Status CopyEngineManager::submit_and_wait(const SGEntry* entries, int count) {
    Status s = submit_scatter_gather(entries, count);
    if (s != GFD_SUCCESS) return s;
    return wait_completion();
}

Status CopyEngineManager::record_event_on_last_stream(gfd_event_t event) {
    if (!initialized_) return GFD_SUCCESS;
    GFD_HIP_CHECK(gfd_hip_event_record(event, streams_[last_channel_]));
    return GFD_SUCCESS;
}

Status CopyEngineManager::make_stream_wait_on_all(gfd_stream_t stream) {
    if (!initialized_ || dirty_mask_ == 0) return GFD_SUCCESS;
    for (uint32_t m = dirty_mask_; m; m &= m - 1) {
        int ch = __builtin_ctz(m);
        GFD_HIP_CHECK(gfd_hip_event_record(events_[ch], streams_[ch]));
        GFD_HIP_CHECK(gfd_hip_stream_wait_event(stream, events_[ch]));
    }
    return GFD_SUCCESS;
}

}  // namespace gfd
