// Emulated gfd_hip_* shim (include/gfd/hip_shim.h) over host memory, plus
// the allocation registry of emu.h.  Streams and events are inert handles:
// the copy engine's SDMA backend (the one under test) never uses them.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

#include "emu.h"
#include "gfd/hip_shim.h"
#include "gfd_capi.h"

namespace emu {
namespace {

struct Alloc {
    size_t size;
    Kind kind;
    uintptr_t agent_base;
};

std::mutex& reg_mu() {
    static std::mutex m;
    return m;
}

std::map<uintptr_t, Alloc>& reg() {
    static std::map<uintptr_t, Alloc> m;
    return m;
}

}  // namespace

void note_alloc(void* p, size_t n, Kind k) {
    std::lock_guard<std::mutex> g(reg_mu());
    reg()[(uintptr_t)p] = Alloc{n, k, (uintptr_t)p};
}

void note_locked(void* p, size_t n, uintptr_t agent_base) {
    std::lock_guard<std::mutex> g(reg_mu());
    reg()[(uintptr_t)p] = Alloc{n, Kind::Locked, agent_base};
}

uintptr_t locked_agent_base(uintptr_t base) {
    std::lock_guard<std::mutex> g(reg_mu());
    auto it = reg().find(base);
    return it == reg().end() ? 0 : it->second.agent_base;
}

void note_free(void* p) {
    std::lock_guard<std::mutex> g(reg_mu());
    reg().erase((uintptr_t)p);
}

bool find_alloc(const void* p, size_t n, Kind k, uintptr_t* base, size_t* size) {
    std::lock_guard<std::mutex> g(reg_mu());
    auto& m = reg();
    auto it = m.upper_bound((uintptr_t)p);
    if (it == m.begin()) return false;
    --it;
    const uintptr_t lo = (uintptr_t)p;
    if (it->second.kind != k || lo < it->first || lo + n > it->first + it->second.size) return false;
    *base = it->first;
    *size = it->second.size;
    return true;
}

}  // namespace emu

namespace {

void* alloc_aligned(size_t bytes) {
    const size_t n = (bytes + 4095) & ~(size_t)4095;
    void* p = std::aligned_alloc(4096, n ? n : 4096);
    if (p) std::memset(p, 0, n ? n : 4096);
    return p;
}

int g_handle = 0;

}  // namespace

namespace {
std::atomic<unsigned> g_zc_launches{0};

void require_gpu_readable(const void* p, size_t n, const char* what) { emu::require_gpu_access(p, n, what); }
}

namespace emu {
// A GPU kernel that reads a host address the runtime has not mapped for the
// GPU takes a page fault (XNACK is off): the emulated kernels end the process
// the same way, so a scenario sees any address handed to them unchecked.
void require_gpu_access(const void* p, size_t n, const char* what) {
    uintptr_t b;
    size_t s;
    if (n == 0 || emu::find_alloc(p, n, emu::Kind::Pinned, &b, &s) || emu::find_alloc(p, n, emu::Kind::Device, &b, &s))
        return;
    std::fprintf(stderr, "emulated GPU fault: %s touches %zu bytes at %p, not pinned or device memory\n", what, n, p);
    std::abort();
}
}  // namespace emu
namespace emu {
unsigned zero_copy_launches() { return g_zc_launches.load(); }
}  // namespace emu

extern "C" {

int gfd_hip_device_count(int* n) {
    *n = 1;
    return 0;
}
int gfd_hip_get_device(int* dev) {
    *dev = 0;
    return 0;
}
int gfd_hip_set_device(int dev) { return dev == 0 ? 0 : 101; }
int gfd_hip_device_synchronize(void) { return 0; }
int gfd_hip_pci_bus_id(char* buf, int len, int dev) {
    if (dev != 0) return 101;
    std::snprintf(buf, (size_t)len, "0000:c1:00.0");
    return 0;
}
int gfd_hip_cu_count(int* n, int) {
    *n = 256;
    return 0;
}
const char* gfd_hip_error_string(int) { return "emulated runtime error"; }

int gfd_hip_host_alloc(void** p, size_t bytes, unsigned) {
    *p = alloc_aligned(bytes);
    if (!*p) return 2;
    emu::note_alloc(*p, bytes, emu::Kind::Pinned);
    return 0;
}
int gfd_hip_host_free(void* p) {
    emu::note_free(p);
    std::free(p);
    return 0;
}
int gfd_hip_host_device_pointer(uint64_t* dptr, void* hptr) {
    *dptr = (uint64_t)(uintptr_t)hptr;
    return 0;
}
int gfd_hip_malloc(void** p, size_t bytes) {
    *p = alloc_aligned(bytes);
    if (!*p) return 2;
    emu::note_alloc(*p, bytes, emu::Kind::Device);
    return 0;
}
int gfd_hip_free(void* p) {
    emu::note_free(p);
    std::free(p);
    return 0;
}

int gfd_hip_stream_create(gfd_stream_t* s) {
    *s = &g_handle;
    return 0;
}
int gfd_hip_stream_destroy(gfd_stream_t) { return 0; }
int gfd_hip_stream_synchronize(gfd_stream_t) { return 0; }
int gfd_hip_event_create(gfd_event_t* e, int) {
    *e = &g_handle;
    return 0;
}
int gfd_hip_event_destroy(gfd_event_t) { return 0; }
int gfd_hip_event_record(gfd_event_t, gfd_stream_t) { return 0; }
int gfd_hip_event_synchronize(gfd_event_t) { return 0; }
int gfd_hip_event_query(gfd_event_t) { return 0; }
int gfd_hip_event_elapsed_ms(float* ms, gfd_event_t, gfd_event_t) {
    *ms = 0.f;
    return 0;
}
int gfd_hip_stream_wait_event(gfd_stream_t, gfd_event_t) { return 0; }

int gfd_hip_memcpy_h2d_async(uint64_t dst, const void* src, size_t bytes, gfd_stream_t) {
    std::memcpy((void*)(uintptr_t)dst, src, bytes);
    return 0;
}
int gfd_hip_memcpy_d2h_async(void* dst, uint64_t src, size_t bytes, gfd_stream_t) {
    std::memcpy(dst, (const void*)(uintptr_t)src, bytes);
    return 0;
}
int gfd_hip_memcpy_h2d(uint64_t dst, const void* src, size_t bytes) {
    std::memcpy((void*)(uintptr_t)dst, src, bytes);
    return 0;
}
int gfd_hip_memcpy_d2h(void* dst, uint64_t src, size_t bytes) {
    std::memcpy(dst, (const void*)(uintptr_t)src, bytes);
    return 0;
}
int gfd_hip_memcpy_d2d(uint64_t dst, uint64_t src, size_t bytes) {
    std::memmove((void*)(uintptr_t)dst, (const void*)(uintptr_t)src, bytes);
    return 0;
}
int gfd_hip_memset_d8(uint64_t dst, int value, size_t bytes) {
    std::memset((void*)(uintptr_t)dst, value, bytes);
    return 0;
}
int gfd_hip_stream_write_u64(gfd_stream_t, uint64_t dst, uint64_t value) {
    __atomic_store_n((uint64_t*)(uintptr_t)dst, value, __ATOMIC_RELEASE);
    return 0;
}
int gfd_hip_pointer_is_device(const void* p) {
    uintptr_t b;
    size_t s;
    return emu::find_alloc(p, 1, emu::Kind::Device, &b, &s) ? 1 : 0;
}
int gfd_hip_device_range(uint64_t ptr, uint64_t* base, uint64_t* size) {
    uintptr_t b;
    size_t s;
    if (!emu::find_alloc((const void*)(uintptr_t)ptr, 1, emu::Kind::Device, &b, &s)) return 0;
    *base = b;
    *size = s;
    return 1;
}

// The Direct path's zero-copy route is a GPU kernel: not emulated.
int gfd_zero_copy_gather(const gfd_sg_entry*, int, void*) { return 801; }

// The zero-copy kernels with host-word completion, run on the calling thread:
// every entry is copied, then the counter is left at 0 and done_value is
// stored with release ordering, as the grid's last wave does.
int gfd_zero_copy_gather_tokens_signal(const uint64_t* src_addrs, void* dst, uint32_t token_size, int num_tokens,
                                       unsigned int* done_counter, uint64_t* done_word, uint64_t done_value,
                                       void*) {
    if (!done_counter || !done_word || num_tokens < 0 || (num_tokens > 0 && (!src_addrs || !dst || !token_size)))
        return 1;
    g_zc_launches++;
    for (int j = 0; j < num_tokens; j++) require_gpu_readable((const void*)(uintptr_t)src_addrs[j], token_size, "zc_gather_tokens");
    for (int j = 0; j < num_tokens; j++)
        std::memcpy((char*)dst + (size_t)j * token_size, (const void*)(uintptr_t)src_addrs[j], token_size);
    __atomic_store_n(done_counter, 0u, __ATOMIC_RELAXED);
    __atomic_store_n(done_word, done_value, __ATOMIC_RELEASE);
    return 0;
}

int gfd_zero_copy_gather_signal(const gfd_sg_entry* entries, int count, unsigned int* done_counter,
                                uint64_t* done_word, uint64_t done_value, void*) {
    if (!done_counter || !done_word || count < 0 || (count > 0 && !entries)) return 1;
    g_zc_launches++;
    for (int i = 0; i < count; i++)
        require_gpu_readable((const void*)(uintptr_t)entries[i].src, entries[i].size, "zc_gather_sg");
    for (int i = 0; i < count; i++)
        std::memcpy((void*)(uintptr_t)entries[i].dst, (const void*)(uintptr_t)entries[i].src, entries[i].size);
    __atomic_store_n(done_counter, 0u, __ATOMIC_RELAXED);
    __atomic_store_n(done_word, done_value, __ATOMIC_RELEASE);
    return 0;
}

int gfd_zero_copy_gather_signal_presliced(const gfd_sg_entry* entries, int count, unsigned int* done_counter,
                                          uint64_t* done_word, uint64_t done_value, void* stream) {
    return gfd_zero_copy_gather_signal(entries, count, done_counter, done_word, done_value, stream);
}

int gfd_zero_copy_target_waves(void) { return 64; }

}  // extern "C"
