// CopyEngineManager (declaration: include/gfd/copy_engine.h).  Channel
// assignment follows src/copy_engine.cpp:103-131 of the reference
// (round-robin for few entries, one contiguous range per channel otherwise);
// completion is tracked with fences instead of per-stream CUDA events.
#include "gfd/copy_engine.h"

#include <cstdlib>
#include <cstring>

#include "sdma.h"

namespace gfd {

namespace {

int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    return (v && *v) ? std::atoi(v) : dflt;
}

}  // namespace

CopyEngineManager::CopyEngineManager() = default;

CopyEngineManager::~CopyEngineManager() { shutdown(); }

Status CopyEngineManager::init(int device, int num_channels) {
    if (initialized_) return GFD_SUCCESS;
    device_ = device;
    num_channels_ = num_channels > 0 ? num_channels : env_int("GFD_CE_CHANNELS", DEFAULT_CE_CHANNELS);
    if (num_channels_ < 1) num_channels_ = 1;
    if (num_channels_ > MAX_CE_CHANNELS) num_channels_ = MAX_CE_CHANNELS;
    GFD_HIP_CHECK(gfd_hip_set_device(device_));
    const char* be = std::getenv("GFD_COPY_BACKEND");
    backend_ = (be && std::strcmp(be, "hip") == 0) ? BACKEND_HIP : BACKEND_SDMA;
    if (backend_ == BACKEND_SDMA) {
        sdma_ = new SdmaQueue();
        int st = sdma_->init(device_, num_channels_, env_int("GFD_SDMA_PIN", 1));
        if (st != 0) {
            GFD_LOG_ERROR("SDMA backend unavailable (status %d); using HIP streams\n", st);
            delete sdma_;
            sdma_ = nullptr;
            backend_ = BACKEND_HIP;
        }
    }
    if (backend_ == BACKEND_HIP) {
        for (int i = 0; i < num_channels_; i++) {
            GFD_HIP_CHECK(gfd_hip_stream_create(&streams_[i]));
            GFD_HIP_CHECK(gfd_hip_event_create(&events_[i], 0));
        }
    }
    next_channel_ = last_channel_ = 0;
    dirty_mask_ = 0;
    initialized_ = true;
    return GFD_SUCCESS;
}

void CopyEngineManager::shutdown() {
    if (!initialized_) return;
    gfd_hip_set_device(device_);
    wait_completion();
    delete sdma_;
    sdma_ = nullptr;
    for (int i = 0; i < MAX_CE_CHANNELS; i++) {
        if (streams_[i]) gfd_hip_stream_destroy(streams_[i]);
        if (events_[i]) gfd_hip_event_destroy(events_[i]);
        streams_[i] = nullptr;
        events_[i] = nullptr;
    }
    initialized_ = false;
}

int CopyEngineManager::num_sdma_engines() const { return sdma_ ? sdma_->num_engines() : 0; }

static_assert(sizeof(CopyEngineManager::CopyTime) == sizeof(SdmaQueue::CopyTime), "copy time layout");

void CopyEngineManager::set_copy_timing(bool on) {
    if (sdma_) sdma_->set_timing(on);
}

size_t CopyEngineManager::read_copy_times(CopyTime* out, size_t max) {
    return sdma_ ? sdma_->read_times(reinterpret_cast<SdmaQueue::CopyTime*>(out), max) : 0;
}

uint64_t CopyEngineManager::copy_clock_ns() const { return sdma_ ? sdma_->now_ns() : 0; }

bool CopyEngineManager::host_source_ok(const void* p, size_t n) { return sdma_ && sdma_->host_source_ok(p, n); }
void CopyEngineManager::last_pinned_range(uintptr_t* lo, uintptr_t* hi) const {
    *lo = *hi = 0;
    if (sdma_) sdma_->last_pinned_range(lo, hi);
}
void CopyEngineManager::forget_pinned_range() {
    if (sdma_) sdma_->forget_pinned_range();
}
void CopyEngineManager::trust_range(const void* p, size_t n) {
    if (sdma_) sdma_->trust_range(p, n);
}
uint32_t CopyEngineManager::sdma_engine_mask() const { return sdma_ ? sdma_->engine_mask() : 0; }

Status CopyEngineManager::pin_context() {
    if (!initialized_) return GFD_SUCCESS;
    GFD_HIP_CHECK(gfd_hip_set_device(device_));
    return GFD_SUCCESS;
}

void CopyEngineManager::unpin_context() {}

Status CopyEngineManager::issue(int ch, DevicePtr dst, const void* src, size_t size) {
    ch %= num_channels_;
    if (backend_ == BACKEND_SDMA) {
        if (!sdma_->host_source_ok(src, size)) {
            // Pageable (or unknown) source: the SDMA engines cannot read it.
            // Let the HIP runtime stage it (synchronous copy).
            static bool warned = false;
            if (!warned) {
                GFD_LOG_INFO("source %p is not pinned host memory: using synchronous hipMemcpy for it\n", src);
                warned = true;
            }
            GFD_HIP_CHECK(gfd_hip_memcpy_h2d(dst, src, size));
            total_bytes_ += (double)size;
            return GFD_SUCCESS;
        }
        int st = sdma_->copy(ch, dst, src, size);
        if (st != 0) {
            GFD_LOG_ERROR("SDMA copy failed (%d)\n", st);
            return st;
        }
    } else {
        GFD_HIP_CHECK(gfd_hip_memcpy_h2d_async(dst, src, size, streams_[ch]));
        dirty_mask_ |= 1u << ch;
        hip_fence_++;
    }
    last_channel_ = ch;
    total_bytes_ += (double)size;
    return GFD_SUCCESS;
}

Status CopyEngineManager::submit_on_channel(int ch, DevicePtr dst, const void* src, size_t size) {
    if (!initialized_) return GFD_SUCCESS;
    Status s = issue(ch, dst, src, size);
    if (s) return s;
    if (backend_ == BACKEND_HIP) GFD_HIP_CHECK(gfd_hip_event_record(events_[last_channel_], streams_[last_channel_]));
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
            Status s = issue(ch, entries[i].dst, entries[i].src, entries[i].size);
            if (s) return s;
            used |= 1u << ch;
        }
    } else {
        int per = (count + num_channels_ - 1) / num_channels_;
        for (int ch = 0; ch < num_channels_; ch++) {
            int b = ch * per;
            if (b >= count) break;
            int e = b + per < count ? b + per : count;
            for (int i = b; i < e; i++) {
                Status s = issue(ch, entries[i].dst, entries[i].src, entries[i].size);
                if (s) return s;
            }
            used |= 1u << ch;
        }
        next_channel_ = 0;
    }
    if (backend_ == BACKEND_HIP)
        for (uint32_t m = used; m; m &= m - 1) {
            int ch = __builtin_ctz(m);
            GFD_HIP_CHECK(gfd_hip_event_record(events_[ch], streams_[ch]));
        }
    total_submissions_++;
    total_entries_ += (uint64_t)count;
    return GFD_SUCCESS;
}

Status CopyEngineManager::submit_after(DevicePtr dst, const void* src, size_t size, uint64_t after_begin,
                                       uint64_t after_end, uint64_t also_after) {
    if (!initialized_) return GFD_SUCCESS;
    if (backend_ == BACKEND_SDMA && sdma_->channels_in_order()) {
        // One engine per channel, each finishing its copies in order: the
        // newest copy of every channel since after_begin stands for all of
        // that channel's, so the write depends on at most channels + 1
        // copies and nothing is waited for on the host.
        uint64_t deps[MAX_CE_CHANNELS + 1];
        int nd = sdma_->channel_tails(after_begin, deps, MAX_CE_CHANNELS);
        if (nd < 0) return -1;
        const uint64_t tail = sdma_->retire();
        if (also_after != kNoFence && also_after >= tail) {
            bool have = false;
            for (int i = 0; i < nd; i++) have |= deps[i] == also_after;
            if (!have) deps[nd++] = also_after;
        }
        int st = sdma_->copy(last_channel_, dst, src, size, nullptr, deps, nd);
        if (st) return st;
    } else if (backend_ == BACKEND_SDMA) {
        // Runtime-chosen engines: no order between copies to lean on.
        uint64_t deps[16];
        int nd = 0;
        const uint64_t tail = sdma_->retire();
        if (after_begin < tail) after_begin = tail;
        const bool extra = also_after != kNoFence && also_after >= tail &&
                           (also_after < after_begin || also_after >= after_end);
        const uint64_t room = extra ? 15 : 16;
        if (after_end > after_begin && after_end - after_begin > room) {
            // Too many to chain on the engine: wait for the older ones here.
            if (sdma_->wait(after_end - room) != 0) return -1;
            after_begin = after_end - room;
        }
        for (uint64_t f = after_begin; f < after_end; f++) deps[nd++] = f;
        if (extra) deps[nd++] = also_after;
        int st = sdma_->copy(last_channel_, dst, src, size, nullptr, deps, nd);
        if (st) return st;
    } else {
        // Same stream order would not cover other channels: wait, then copy.
        Status s = wait_completion();
        if (s) return s;
        GFD_HIP_CHECK(gfd_hip_memcpy_h2d_async(dst, src, size, streams_[0]));
        GFD_HIP_CHECK(gfd_hip_event_record(events_[0], streams_[0]));
        dirty_mask_ |= 1u;
        hip_fence_++;
    }
    total_submissions_++;
    return GFD_SUCCESS;
}

uint64_t CopyEngineManager::fence() const { return sdma_ ? sdma_->issued() : hip_fence_; }

bool CopyEngineManager::fence_done(uint64_t f) {
    if (sdma_) return sdma_->done(f);
    for (uint32_t m = dirty_mask_; m; m &= m - 1)
        if (gfd_hip_event_query(events_[__builtin_ctz(m)]) == 1) return false;
    return true;
}

Status CopyEngineManager::wait_fence(uint64_t f) {
    if (sdma_) return sdma_->wait(f);
    return wait_completion();
}

Status CopyEngineManager::wait_completion() {
    if (!initialized_) return GFD_SUCCESS;
    if (sdma_) return sdma_->wait_all();
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
    if (sdma_) return sdma_->wait_all();
    GFD_HIP_CHECK(gfd_hip_event_record(event, streams_[last_channel_]));
    return GFD_SUCCESS;
}

Status CopyEngineManager::make_stream_wait_on_all(gfd_stream_t stream) {
    if (!initialized_) return GFD_SUCCESS;
    if (sdma_) return sdma_->wait_all();
    for (uint32_t m = dirty_mask_; m; m &= m - 1) {
        int ch = __builtin_ctz(m);
        GFD_HIP_CHECK(gfd_hip_event_record(events_[ch], streams_[ch]));
        GFD_HIP_CHECK(gfd_hip_stream_wait_event(stream, events_[ch]));
    }
    return GFD_SUCCESS;
}

}  // namespace gfd
