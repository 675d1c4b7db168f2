// Emulated HSA runtime: the subset SdmaQueue (gfd_amd/csrc/sdma.cpp) calls.
// See emu.h for the copy-engine model.
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>
#include <vector>

#include "emu.h"

namespace {

constexpr uint64_t kCpuAgent = 0x1000, kGpuAgent = 0x2000;

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

long env_long(const char* name, long dflt) {
    const char* v = std::getenv(name);
    return (v && *v) ? std::atol(v) : dflt;
}

struct Signal {
    std::atomic<int64_t> value;
    uint64_t start_ns = 0, end_ns = 0;
    explicit Signal(int64_t v) : value(v) {}
};

Signal* S(hsa_signal_t s) { return reinterpret_cast<Signal*>(s.handle); }

struct Packet {
    void* dst;
    const void* src;
    size_t size;
    std::vector<Signal*> deps;
    Signal* done;
    uint64_t id;
};

struct Engine {
    std::mutex mu;
    std::condition_variable cv;
    std::deque<Packet> ring;
    std::thread th;
    int index = 0;
};

struct Runtime {
    std::mutex mu;
    int refs = 0;
    std::atomic<bool> stop{false};  // written under each engine's lock in turn, read under another's
    std::vector<Engine*> engines;
    std::atomic<uint64_t> next_id{0};
    std::atomic<unsigned> rr{0};
    long copy_ns = 0, ps_per_byte = 0, stall_ms = 5000;
    bool profiling = false;
};

Runtime& rt() {
    static Runtime r;
    return r;
}

void spin_for(uint64_t ns) {
    if (!ns) return;
    const uint64_t end = now_ns() + ns;
    while (now_ns() < end) {
    }
}

void engine_loop(Engine* e) {
    Runtime& r = rt();
    for (;;) {
        Packet p;
        {
            std::unique_lock<std::mutex> g(e->mu);
            e->cv.wait(g, [&] { return r.stop.load() || !e->ring.empty(); });
            if (e->ring.empty()) return;
            p = e->ring.front();  // stays at the head while it executes
        }
        for (Signal* d : p.deps) {
            const uint64_t t0 = now_ns();
            uint64_t spins = 0;
            while (d->value.load(std::memory_order_acquire) != 0) {
                if ((++spins & 1023) == 0) {
                    std::this_thread::yield();
                    if (now_ns() - t0 > (uint64_t)r.stall_ms * 1000000ull) {
                        std::fprintf(stderr,
                                     "hsa_emu: engine %d stalled %ld ms at packet %llu polling signal %p "
                                     "(value %lld)\n",
                                     e->index, r.stall_ms, (unsigned long long)p.id, (void*)d,
                                     (long long)d->value.load());
                        std::fflush(stderr);
                        _exit(emu::kStallExit);
                    }
                }
            }
        }
        const uint64_t t1 = now_ns();
        if (p.size == 8 && ((uintptr_t)p.dst & 7) == 0) {
            uint64_t v;
            std::memcpy(&v, p.src, 8);
            __atomic_store_n((uint64_t*)p.dst, v, __ATOMIC_RELEASE);
        } else {
            std::memcpy(p.dst, p.src, p.size);
        }
        spin_for((uint64_t)r.copy_ns + (uint64_t)((double)p.size * (double)r.ps_per_byte / 1000.0));
        if (p.done) {
            p.done->start_ns = t1;
            p.done->end_ns = now_ns();
            p.done->value.fetch_sub(1, std::memory_order_acq_rel);
        }
        std::lock_guard<std::mutex> g(e->mu);
        e->ring.pop_front();
    }
}

hsa_status_t enqueue(int engine, void* dst, const void* src, size_t size, uint32_t ndeps, const hsa_signal_t* deps,
                     hsa_signal_t done) {
    Runtime& r = rt();
    if (engine < 0 || engine >= (int)r.engines.size()) return HSA_STATUS_ERROR_INVALID_ARGUMENT;
    Packet p{dst, src, size, {}, done.handle ? S(done) : nullptr, r.next_id.fetch_add(1)};
    for (uint32_t i = 0; i < ndeps; i++) p.deps.push_back(S(deps[i]));
    Engine* e = r.engines[(size_t)engine];
    {
        std::lock_guard<std::mutex> g(e->mu);
        e->ring.push_back(std::move(p));
    }
    e->cv.notify_one();
    return HSA_STATUS_SUCCESS;
}

}  // namespace

extern "C" {

hsa_status_t HSA_API hsa_init() {
    Runtime& r = rt();
    std::lock_guard<std::mutex> g(r.mu);
    if (r.refs++ > 0) return HSA_STATUS_SUCCESS;
    r.stop.store(false);
    r.copy_ns = env_long("GFD_EMU_COPY_NS", 300);
    r.ps_per_byte = env_long("GFD_EMU_PS_PER_BYTE", 20);
    r.stall_ms = env_long("GFD_EMU_STALL_MS", 5000);
    const long n = env_long("GFD_EMU_ENGINES", 4);
    for (long i = 0; i < n && i < 16; i++) {
        Engine* e = new Engine();
        e->index = (int)i;
        r.engines.push_back(e);
        e->th = std::thread(engine_loop, e);
    }
    return HSA_STATUS_SUCCESS;
}

hsa_status_t HSA_API hsa_shut_down() {
    Runtime& r = rt();
    std::lock_guard<std::mutex> g(r.mu);
    if (r.refs == 0) return HSA_STATUS_ERROR_NOT_INITIALIZED;
    if (--r.refs > 0) return HSA_STATUS_SUCCESS;
    for (Engine* e : r.engines) {
        {
            std::lock_guard<std::mutex> ge(e->mu);
            r.stop.store(true);
        }
        e->cv.notify_all();
    }
    for (Engine* e : r.engines) {
        e->th.join();
        delete e;
    }
    r.engines.clear();
    return HSA_STATUS_SUCCESS;
}

hsa_status_t HSA_API hsa_system_get_info(hsa_system_info_t attribute, void* value) {
    Runtime& r = rt();
    switch (attribute) {
        case HSA_SYSTEM_INFO_VERSION_MAJOR:
            if (r.refs == 0) return HSA_STATUS_ERROR_NOT_INITIALIZED;
            *(uint16_t*)value = 1;
            return HSA_STATUS_SUCCESS;
        case HSA_SYSTEM_INFO_TIMESTAMP_FREQUENCY:
            *(uint64_t*)value = 1000000000ull;
            return HSA_STATUS_SUCCESS;
        case HSA_SYSTEM_INFO_TIMESTAMP:
            *(uint64_t*)value = now_ns();
            return HSA_STATUS_SUCCESS;
        default:
            return HSA_STATUS_ERROR_INVALID_ARGUMENT;
    }
}

hsa_status_t HSA_API hsa_iterate_agents(hsa_status_t (*callback)(hsa_agent_t agent, void* data), void* data) {
    hsa_agent_t a;
    a.handle = kCpuAgent;
    hsa_status_t st = callback(a, data);
    if (st != HSA_STATUS_SUCCESS) return st;
    a.handle = kGpuAgent;
    return callback(a, data);
}

hsa_status_t HSA_API hsa_agent_get_info(hsa_agent_t agent, hsa_agent_info_t attribute, void* value) {
    if ((int)attribute == (int)HSA_AGENT_INFO_DEVICE) {
        *(hsa_device_type_t*)value = agent.handle == kGpuAgent ? HSA_DEVICE_TYPE_GPU : HSA_DEVICE_TYPE_CPU;
        return HSA_STATUS_SUCCESS;
    }
    if ((int)attribute == (int)HSA_AMD_AGENT_INFO_BDFID) {
        *(uint32_t*)value = 0xc1u << 8;  // matches the emulated shim's bus id 0000:c1:00.0
        return HSA_STATUS_SUCCESS;
    }
    if ((int)attribute == (int)HSA_AMD_AGENT_INFO_DOMAIN) {
        *(uint32_t*)value = 0;
        return HSA_STATUS_SUCCESS;
    }
    return HSA_STATUS_ERROR_INVALID_ARGUMENT;
}

hsa_status_t HSA_API hsa_amd_memory_copy_engine_status(hsa_agent_t, hsa_agent_t, uint32_t* engine_ids_mask) {
    const size_t n = rt().engines.size();
    *engine_ids_mask = n >= 32 ? 0xFFFFFFFFu : ((1u << n) - 1u);
    return HSA_STATUS_SUCCESS;
}

hsa_status_t HSA_API hsa_amd_signal_create(hsa_signal_value_t initial_value, uint32_t, const hsa_agent_t*, uint64_t,
                                           hsa_signal_t* signal) {
    signal->handle = (uint64_t)(uintptr_t) new Signal(initial_value);
    return HSA_STATUS_SUCCESS;
}

hsa_status_t HSA_API hsa_signal_destroy(hsa_signal_t signal) {
    delete S(signal);
    return HSA_STATUS_SUCCESS;
}

void HSA_API hsa_signal_store_relaxed(hsa_signal_t signal, hsa_signal_value_t value) {
    S(signal)->value.store(value, std::memory_order_relaxed);
}

hsa_signal_value_t HSA_API hsa_signal_load_scacquire(hsa_signal_t signal) {
    return S(signal)->value.load(std::memory_order_acquire);
}

hsa_signal_value_t HSA_API hsa_signal_wait_scacquire(hsa_signal_t signal, hsa_signal_condition_t condition,
                                                     hsa_signal_value_t compare_value, uint64_t, hsa_wait_state_t) {
    Signal* s = S(signal);
    for (;;) {
        const hsa_signal_value_t v = s->value.load(std::memory_order_acquire);
        bool ok = false;
        switch (condition) {
            case HSA_SIGNAL_CONDITION_EQ: ok = v == compare_value; break;
            case HSA_SIGNAL_CONDITION_NE: ok = v != compare_value; break;
            case HSA_SIGNAL_CONDITION_LT: ok = v < compare_value; break;
            case HSA_SIGNAL_CONDITION_GTE: ok = v >= compare_value; break;
        }
        if (ok) return v;
        std::this_thread::yield();
    }
}

hsa_status_t HSA_API hsa_amd_memory_async_copy_on_engine(void* dst, hsa_agent_t, const void* src, hsa_agent_t,
                                                         size_t size, uint32_t num_dep_signals,
                                                         const hsa_signal_t* dep_signals,
                                                         hsa_signal_t completion_signal,
                                                         hsa_amd_sdma_engine_id_t engine_id, bool) {
    const uint32_t id = (uint32_t)engine_id;
    if (id == 0 || (id & (id - 1))) return HSA_STATUS_ERROR_INVALID_ARGUMENT;
    // Copies on pinned engines depend on at most one copy per channel plus
    // the previous flag write (CopyEngineManager::submit_after): at most
    // MAX_CE_CHANNELS + 1 = 9 signals.
    if (num_dep_signals > 9) {
        std::fprintf(stderr, "emulated SDMA: copy with %u dependency signals (bound 9)\n", num_dep_signals);
        std::abort();
    }
    return enqueue(__builtin_ctz(id), dst, src, size, num_dep_signals, dep_signals, completion_signal);
}

hsa_status_t HSA_API hsa_amd_memory_async_copy(void* dst, hsa_agent_t, const void* src, hsa_agent_t, size_t size,
                                               uint32_t num_dep_signals, const hsa_signal_t* dep_signals,
                                               hsa_signal_t completion_signal) {
    Runtime& r = rt();
    const int e = (int)(r.rr.fetch_add(1) % (unsigned)r.engines.size());
    return enqueue(e, dst, src, size, num_dep_signals, dep_signals, completion_signal);
}

hsa_status_t HSA_API hsa_amd_pointer_info(const void* ptr, hsa_amd_pointer_info_t* info, void* (*)(size_t),
                                          uint32_t* num_agents_accessible, hsa_agent_t** accessible) {
    if (num_agents_accessible) *num_agents_accessible = 0;
    if (accessible) *accessible = nullptr;
    uintptr_t base = 0;
    size_t size = 0;
    if (emu::find_alloc(ptr, 1, emu::Kind::Pinned, &base, &size)) {
        info->type = HSA_EXT_POINTER_TYPE_HSA;
        info->hostBaseAddress = (void*)base;
        info->agentBaseAddress = (void*)base;
        info->sizeInBytes = size;
    } else if (emu::find_alloc(ptr, 1, emu::Kind::Locked, &base, &size)) {
        info->type = HSA_EXT_POINTER_TYPE_LOCKED;
        info->hostBaseAddress = (void*)base;
        info->agentBaseAddress = (void*)emu::locked_agent_base(base);
        info->sizeInBytes = size;
    } else if (emu::find_alloc(ptr, 1, emu::Kind::Device, &base, &size)) {
        info->type = HSA_EXT_POINTER_TYPE_HSA;
        info->hostBaseAddress = nullptr;
        info->agentBaseAddress = (void*)base;
        info->sizeInBytes = size;
    } else {
        info->type = HSA_EXT_POINTER_TYPE_UNKNOWN;
    }
    return HSA_STATUS_SUCCESS;
}

hsa_status_t HSA_API hsa_amd_profiling_async_copy_enable(bool enable) {
    rt().profiling = enable;
    return HSA_STATUS_SUCCESS;
}

hsa_status_t HSA_API hsa_amd_profiling_get_async_copy_time(hsa_signal_t signal,
                                                           hsa_amd_profiling_async_copy_time_t* time) {
    time->start = S(signal)->start_ns;
    time->end = S(signal)->end_ns;
    return HSA_STATUS_SUCCESS;
}

}  // extern "C"
