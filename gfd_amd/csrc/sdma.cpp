// SdmaQueue (see sdma.h).
#include "sdma.h"

#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <immintrin.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "gfd/hip_shim.h"
#include "gfd/log.h"

namespace gfd {

namespace {

// In-flight copies before the issuer waits.  The signals are polled, never
// slept on, so they are created without interrupt events: the driver's
// per-process event pool is small and HIP and profilers need it too.
constexpr size_t kRing = 1024;

struct AgentSearch {
    uint32_t bdf;
    uint32_t domain;
    hsa_agent_t gpu{0};
    hsa_agent_t cpu{0};
    bool have_gpu = false;
    bool have_cpu = false;
    int gpu_index = 0;
    int want_index = 0;
    hsa_agent_t nth_gpu{0};
    bool have_nth = false;
};

hsa_status_t visit_agent(hsa_agent_t a, void* p) {
    AgentSearch* s = (AgentSearch*)p;
    hsa_device_type_t type;
    if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &type) != HSA_STATUS_SUCCESS) return HSA_STATUS_SUCCESS;
    if (type == HSA_DEVICE_TYPE_CPU && !s->have_cpu) {
        s->cpu = a;
        s->have_cpu = true;
    } else if (type == HSA_DEVICE_TYPE_GPU) {
        uint32_t bdf = 0, dom = 0;
        hsa_agent_get_info(a, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_BDFID, &bdf);
        hsa_agent_get_info(a, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_DOMAIN, &dom);
        if (bdf == s->bdf && dom == s->domain && !s->have_gpu) {
            s->gpu = a;
            s->have_gpu = true;
        }
        if (s->gpu_index == s->want_index) {
            s->nth_gpu = a;
            s->have_nth = true;
        }
        s->gpu_index++;
    }
    return HSA_STATUS_SUCCESS;
}

inline hsa_signal_t sig(uint64_t h) {
    hsa_signal_t s;
    s.handle = h;
    return s;
}

}  // namespace

int find_hsa_agents(int device, uint64_t* gpu_agent, uint64_t* cpu_agent) {
    AgentSearch s;
    s.want_index = device;
    char bus[64] = {0};
    unsigned dom = 0, b = 0, d = 0, f = 0;
    if (gfd_hip_pci_bus_id(bus, sizeof(bus), device) == 0 && std::sscanf(bus, "%x:%x:%x.%x", &dom, &b, &d, &f) == 4) {
        s.bdf = (b << 8) | (d << 3) | f;
        s.domain = dom;
    } else {
        s.bdf = 0xFFFFFFFFu;
        s.domain = 0xFFFFFFFFu;
    }
    hsa_iterate_agents(visit_agent, &s);
    if (!s.have_cpu || !(s.have_gpu || s.have_nth)) return (int)HSA_STATUS_ERROR_INVALID_AGENT;
    *gpu_agent = s.have_gpu ? s.gpu.handle : s.nth_gpu.handle;
    *cpu_agent = s.cpu.handle;
    return 0;
}

SdmaQueue::SdmaQueue() = default;

SdmaQueue::~SdmaQueue() {
    if (!inited_) return;
    wait_all();
    for (uint64_t h : signals_)
        if (h) hsa_signal_destroy(sig(h));
    if (own_hsa_) hsa_shut_down();
}

int SdmaQueue::init(int device, int channels, int pin_engines) {
    if (inited_) return 0;
    // HIP has normally initialised the runtime already; only take a reference
    // of our own when it has not.
    uint16_t major = 0;
    if (hsa_system_get_info(HSA_SYSTEM_INFO_VERSION_MAJOR, &major) != HSA_STATUS_SUCCESS) {
        hsa_status_t st0 = hsa_init();
        if (st0 != HSA_STATUS_SUCCESS) return (int)st0;
        own_hsa_ = true;
    }
    hsa_status_t st = HSA_STATUS_SUCCESS;
    if (find_hsa_agents(device, &gpu_agent_, &cpu_agent_) != 0) {
        GFD_LOG_ERROR("SDMA: HSA agents for device %d not found\n", device);
        if (own_hsa_) hsa_shut_down();
        own_hsa_ = false;
        return (int)HSA_STATUS_ERROR_INVALID_AGENT;
    }
    hsa_agent_t gpu{gpu_agent_}, cpu{cpu_agent_};
    engine_mask_ = 0;
    hsa_amd_memory_copy_engine_status(gpu, cpu, &engine_mask_);
    engines_.clear();
    for (uint32_t m = engine_mask_; m; m &= m - 1) engines_.push_back(m & (~m + 1));
    channels_ = channels > 0 ? channels : 1;
    pin_ = pin_engines && !engines_.empty();
    signals_.assign(kRing, 0);
    for (size_t i = 0; i < kRing; i++) {
        hsa_signal_t h;
        // GPU_ONLY: a plain memory signal without an interrupt event; the
        // host still reads it (load / spin-wait), it just is never woken.
        st = hsa_amd_signal_create(0, 0, nullptr, HSA_AMD_SIGNAL_AMD_GPU_ONLY, &h);
        if (st != HSA_STATUS_SUCCESS) return (int)st;
        signals_[i] = h.handle;
    }
    slot_bytes_.assign(kRing, 0);
    slot_channel_.assign(kRing, 0);
    waiter_.assign(kRing, 0);
    ch_last_.assign((size_t)channels_, 0);
    uint64_t freq = 0;
    if (hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY, &freq) == HSA_STATUS_SUCCESS && freq)
        tick_ns_ = 1e9 / (double)freq;
    next_seq_ = tail_ = 0;
    error_ = 0;
    inited_ = true;
    GFD_LOG_DEBUG("SDMA: engines mask 0x%x, %d channel(s), pinned=%d\n", engine_mask_, channels_, (int)pin_);
    return 0;
}

int SdmaQueue::channel_tails(uint64_t begin, uint64_t* deps, int max_deps) {
    retire();
    int n = 0;
    for (uint64_t last : ch_last_)
        if (last > 0 && last - 1 >= begin && last - 1 >= tail_) {
            if (n == max_deps) return -1;  // more channels than the caller has room for
            deps[n++] = last - 1;
        }
    return n;
}

uint64_t SdmaQueue::retire() {
    while (tail_ < next_seq_) {
        const size_t slot = tail_ % kRing;
        hsa_signal_value_t v = hsa_signal_load_scacquire(sig(signals_[slot]));
        if (v > 0) break;
        if (v < 0) error_ = -1;
        if (timing_.load(std::memory_order_acquire)) {
            hsa_amd_profiling_async_copy_time_t t{};
            if (hsa_amd_profiling_get_async_copy_time(sig(signals_[slot]), &t) == HSA_STATUS_SUCCESS &&
                t.end >= t.start && t.start != 0) {
                const uint32_t ch = slot_channel_[slot];
                CopyTime c{tail_, slot_bytes_[slot], (uint64_t)((double)t.start * tick_ns_),
                           (uint64_t)((double)t.end * tick_ns_), ch,
                           pin_ ? engines_[(size_t)ch % engines_.size()] : 0u};
                std::lock_guard<std::mutex> g(times_mu_);
                if (times_.size() < (1u << 20)) times_.push_back(c);
            }
        }
        tail_++;
    }
    return tail_;
}

void SdmaQueue::set_timing(bool on) {
    // Callable from any thread: only the runtime switch and an atomic flag
    // change.  Copies issued while profiling was off return no timestamps
    // and are skipped when they retire.
    if (!inited_ || on == timing_.load(std::memory_order_relaxed)) return;
    if (hsa_amd_profiling_async_copy_enable(on) == HSA_STATUS_SUCCESS) timing_.store(on, std::memory_order_release);
}

size_t SdmaQueue::read_times(CopyTime* out, size_t max) {
    // Only copies already retired by their issuing thread are returned.
    std::lock_guard<std::mutex> g(times_mu_);
    const size_t n = times_.size() < max ? times_.size() : max;
    for (size_t i = 0; i < n; i++) out[i] = times_[i];
    times_.erase(times_.begin(), times_.begin() + (ptrdiff_t)n);
    return n;
}

uint64_t SdmaQueue::now_ns() const {
    uint64_t ts = 0;
    hsa_system_get_info(HSA_SYSTEM_INFO_TIMESTAMP, &ts);
    return (uint64_t)((double)ts * tick_ns_);
}

int SdmaQueue::wait(uint64_t seq_end) {
    if (seq_end > next_seq_) seq_end = next_seq_;
    while (retire() < seq_end) {
        hsa_signal_t s = sig(signals_[tail_ % kRing]);
        hsa_signal_wait_scacquire(s, HSA_SIGNAL_CONDITION_LT, 1, UINT64_MAX, HSA_WAIT_STATE_ACTIVE);
    }
    return error_ ? -1 : 0;
}

void SdmaQueue::trust_range(const void* p, size_t n) {
    if (!p || n == 0 || ntrusted_ == kMaxTrusted) return;
    trusted_lo_[ntrusted_] = (uintptr_t)p;
    trusted_hi_[ntrusted_] = (uintptr_t)p + n;
    ntrusted_++;
}

bool SdmaQueue::host_source_ok(const void* p, size_t n) {
    const uintptr_t lo = (uintptr_t)p, hi = lo + n;
    for (int i = 0; i < ntrusted_; i++)
        if (lo >= trusted_lo_[i] && hi <= trusted_hi_[i]) return true;
    if (lo >= ok_lo_ && hi <= ok_hi_) return true;
    hsa_amd_pointer_info_t info;
    std::memset(&info, 0, sizeof(info));
    info.size = sizeof(info);
    if (hsa_amd_pointer_info(const_cast<void*>(p), &info, nullptr, nullptr, nullptr) != HSA_STATUS_SUCCESS)
        return false;
    if (info.type != HSA_EXT_POINTER_TYPE_HSA && info.type != HSA_EXT_POINTER_TYPE_LOCKED) return false;
    // Registered (locked) memory can be mapped for the GPU at another address
    // than the host's.  Copies and kernels here are given host addresses, so
    // such a range is not a legal source: the caller then copies it another way.
    if (info.type == HSA_EXT_POINTER_TYPE_LOCKED && info.agentBaseAddress != info.hostBaseAddress) return false;
    const uintptr_t base = (uintptr_t)info.hostBaseAddress;
    if (!base || lo < base || hi > base + info.sizeInBytes) return false;
    ok_lo_ = base;
    ok_hi_ = base + info.sizeInBytes;
    return true;
}

int SdmaQueue::copy(int channel, uint64_t dst, const void* src, size_t bytes, uint64_t* seq,
                    const uint64_t* deps, int ndeps) {
    if (!inited_) return (int)HSA_STATUS_ERROR_NOT_INITIALIZED;
    // Reuse of a ring slot requires its previous copy to be finished.
    if (next_seq_ - tail_ >= kRing) {
        if (wait(next_seq_ - kRing + 1) != 0) return -1;
    }
    const uint64_t s = next_seq_;
    // A copy that depends on this slot's previous occupant may not have
    // polled its signal yet (it can sit behind other copies on its engine).
    // Resetting the signal now would make it wait for this new copy instead,
    // which may be queued behind it on the same engine: wait for it first.
    // It can finish: its dependency, the previous occupant, has completed.
    const uint64_t w = waiter_[s % kRing];
    if (w > tail_ && wait(w) != 0) return -1;
    waiter_[s % kRing] = 0;
    hsa_signal_t cs = sig(signals_[s % kRing]);
    hsa_signal_store_relaxed(cs, 1);
    hsa_signal_t dep_sigs[16];
    size_t dep_slots[16];
    uint32_t nd = 0;
    for (int i = 0; i < ndeps && nd < 16; i++)
        if (deps[i] >= tail_ && deps[i] < s) {
            dep_slots[nd] = deps[i] % kRing;
            dep_sigs[nd++] = sig(signals_[deps[i] % kRing]);
        }
    hsa_agent_t gpu{gpu_agent_}, cpu{cpu_agent_};
    hsa_status_t st;
    if (pin_) {
        const uint32_t eng = engines_[(size_t)channel % engines_.size()];
        st = hsa_amd_memory_async_copy_on_engine((void*)(uintptr_t)dst, gpu, src, cpu, bytes, nd,
                                                 nd ? dep_sigs : nullptr, cs, (hsa_amd_sdma_engine_id_t)eng, true);
    } else {
        st = hsa_amd_memory_async_copy((void*)(uintptr_t)dst, gpu, src, cpu, bytes, nd, nd ? dep_sigs : nullptr, cs);
    }
    if (st != HSA_STATUS_SUCCESS) {
        hsa_signal_store_relaxed(cs, 0);
        return (int)st;
    }
    for (uint32_t i = 0; i < nd; i++) waiter_[dep_slots[i]] = s + 1;
    ch_last_[(size_t)channel % ch_last_.size()] = s + 1;
    slot_bytes_[s % kRing] = bytes;
    slot_channel_[s % kRing] = (uint32_t)channel;
    next_seq_ = s + 1;
    if (seq) *seq = s;
    return 0;
}

}  // namespace gfd
