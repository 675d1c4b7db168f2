// C-ABI entry points (declarations: include/gfd_capi.h).  Thin wrappers over
// the C++ API; no logic of their own beyond argument checks, error capture and
// the measurement loops of the gfd_bench_* helpers.
#include "gfd_capi.h"

#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <string>
#include <vector>

#include "gather_engine.h"
#include "sdma.h"
#include "gfd/cpu_polling.h"
#include "capi_error.h"
#include "gfd/hip_shim.h"
#include "gfd/sg_task_queue.h"
#include "gfd/staging_pool.h"

static_assert(sizeof(gfd_sg_entry) == sizeof(gfd::SGEntry), "gfd_sg_entry must match gfd::SGEntry");

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* what) {
    g_last_error = std::string(what) + ": " + gfd_hip_error_string(code);
    return code;
}

#define CAPI_CHECK(call, what)               \
    do {                                     \
        int e_ = (call);                     \
        if (e_ != 0) return fail(e_, what);  \
    } while (0)

gfd::CpuPollingThread* P(gfd_poller_t p) { return static_cast<gfd::CpuPollingThread*>(p); }

double elapsed_us(std::chrono::steady_clock::time_point a, std::chrono::steady_clock::time_point b) {
    return std::chrono::duration<double, std::micro>(b - a).count();
}


// Time `launch(stream)` warmup + iters times: wall clock launch -> sync and
// HIP events around the launch on its stream.
template <typename Launch>
int bench_kernel(Launch launch, int warmup, int iters, double* wall_us, double* event_us, const char* what) {
    gfd_stream_t s = nullptr;
    gfd_event_t a = nullptr, b = nullptr;
    int rc = gfd_hip_stream_create(&s);
    if (!rc) rc = gfd_hip_event_create(&a, 1);
    if (!rc) rc = gfd_hip_event_create(&b, 1);
    for (int it = -warmup; it < iters && !rc; it++) {
        auto t0 = std::chrono::steady_clock::now();
        rc = gfd_hip_event_record(a, s);
        if (!rc) rc = launch(s);
        if (!rc) rc = gfd_hip_event_record(b, s);
        if (!rc) rc = gfd_hip_stream_synchronize(s);
        auto t1 = std::chrono::steady_clock::now();
        float ms = 0;
        if (!rc) rc = gfd_hip_event_elapsed_ms(&ms, a, b);
        if (it >= 0 && !rc) {
            wall_us[it] = elapsed_us(t0, t1);
            if (event_us) event_us[it] = ms * 1000.0;
        }
    }
    if (a) gfd_hip_event_destroy(a);
    if (b) gfd_hip_event_destroy(b);
    if (s) gfd_hip_stream_destroy(s);
    return rc ? fail(rc, what) : 0;
}

}  // namespace

void gfd_internal_set_error(const char* what) { g_last_error = what ? what : ""; }

extern "C" {

const char* gfd_version(void) { return "gfd-amd 0.1.0 (gfx950)"; }
const char* gfd_last_error(void) { return g_last_error.c_str(); }

int gfd_device_count(int* n) { CAPI_CHECK(gfd_hip_device_count(n), "hipGetDeviceCount"); return 0; }
int gfd_set_device(int dev) { CAPI_CHECK(gfd_hip_set_device(dev), "hipSetDevice"); return 0; }
int gfd_device_synchronize(void) { CAPI_CHECK(gfd_hip_device_synchronize(), "hipDeviceSynchronize"); return 0; }

int gfd_host_alloc(void** p, size_t bytes, unsigned flags) {
    CAPI_CHECK(gfd_hip_host_alloc(p, bytes, flags), "hipHostMalloc");
    return 0;
}
int gfd_host_free(void* p) { CAPI_CHECK(gfd_hip_host_free(p), "hipHostFree"); return 0; }
int gfd_device_alloc(void** p, size_t bytes) { CAPI_CHECK(gfd_hip_malloc(p, bytes), "hipMalloc"); return 0; }
int gfd_device_free(void* p) { CAPI_CHECK(gfd_hip_free(p), "hipFree"); return 0; }
int gfd_memcpy_h2d(void* dst, const void* src, size_t n) {
    CAPI_CHECK(gfd_hip_memcpy_h2d((uint64_t)(uintptr_t)dst, src, n), "hipMemcpy H2D");
    return 0;
}
int gfd_memcpy_d2h(void* dst, const void* src, size_t n) {
    CAPI_CHECK(gfd_hip_memcpy_d2h(dst, (uint64_t)(uintptr_t)src, n), "hipMemcpy D2H");
    return 0;
}
int gfd_memcpy_d2d(void* dst, const void* src, size_t n) {
    CAPI_CHECK(gfd_hip_memcpy_d2d((uint64_t)(uintptr_t)dst, (uint64_t)(uintptr_t)src, n), "hipMemcpy D2D");
    CAPI_CHECK(gfd_hip_device_synchronize(), "hipDeviceSynchronize");  // device-to-device copies may return early
    return 0;
}
int gfd_memset_device(void* dst, int value, size_t n) {
    // hipMemset of device memory may return before the fill has run (as
    // cudaMemset may); SDMA copies issued next by submit_direct are not
    // ordered after it, so wait.
    CAPI_CHECK(gfd_hip_memset_d8((uint64_t)(uintptr_t)dst, value, n), "hipMemset");
    CAPI_CHECK(gfd_hip_device_synchronize(), "hipDeviceSynchronize");
    return 0;
}
int gfd_stream_create(void** s) { CAPI_CHECK(gfd_hip_stream_create(s), "hipStreamCreate"); return 0; }
int gfd_stream_destroy(void* s) { CAPI_CHECK(gfd_hip_stream_destroy(s), "hipStreamDestroy"); return 0; }
int gfd_stream_synchronize(void* s) { CAPI_CHECK(gfd_hip_stream_synchronize(s), "hipStreamSynchronize"); return 0; }
int gfd_event_create(void** e) { CAPI_CHECK(gfd_hip_event_create(e, 1), "hipEventCreate"); return 0; }
int gfd_event_destroy(void* e) { CAPI_CHECK(gfd_hip_event_destroy(e), "hipEventDestroy"); return 0; }
int gfd_event_record(void* e, void* s) { CAPI_CHECK(gfd_hip_event_record(e, s), "hipEventRecord"); return 0; }
int gfd_event_synchronize(void* e) { CAPI_CHECK(gfd_hip_event_synchronize(e), "hipEventSynchronize"); return 0; }
int gfd_event_elapsed_ms(float* ms, void* a, void* b) {
    CAPI_CHECK(gfd_hip_event_elapsed_ms(ms, a, b), "hipEventElapsedTime");
    return 0;
}

// ---- CpuPollingThread ----

gfd_poller_t gfd_poller_create(void* queue, void* gpu_base, void* cpu_base, size_t total_cpu_size, int use_ce,
                               int numa_node, int core_offset, int num_ce_channels, int exclusive_core_base,
                               int exclusive_core_count) {
    try {
        return new gfd::CpuPollingThread((gfd::DescriptorQueue*)queue, gpu_base, cpu_base, total_cpu_size,
                                         use_ce != 0, numa_node, core_offset, num_ce_channels,
                                         exclusive_core_base, exclusive_core_count);
    } catch (const std::exception& ex) {
        g_last_error = ex.what();
        return nullptr;
    }
}

void gfd_poller_destroy(gfd_poller_t p) { delete P(p); }

int gfd_poller_init_copy_engine(gfd_poller_t p) {
    if (!p) return fail(1, "null poller");
    if (!P(p)->init_copy_engine()) {
        g_last_error = "init_copy_engine failed";
        return -1;
    }
    return 0;
}

int gfd_poller_init_direct_ce(gfd_poller_t p) {
    if (!p) return fail(1, "null poller");
    if (!P(p)->init_direct_ce()) {
        g_last_error = "init_direct_ce failed";
        return -1;
    }
    return 0;
}

double gfd_poller_submit_direct(gfd_poller_t p, const gfd_sg_entry* entries, int count) {
    if (!p) return -1.0;
    return P(p)->submit_direct(reinterpret_cast<const gfd::SGEntry*>(entries), count);
}

void gfd_poller_set_tiled_queue(gfd_poller_t p, void* tq) {
    if (p) P(p)->set_tiled_queue((gfd::TiledQueue*)tq);
}
int gfd_poller_set_sg_task_queue(gfd_poller_t p, void* sq) {
    if (!p) return fail(1, "null poller");
    P(p)->set_sg_task_queue((gfd::SGTaskQueue*)sq);
    if (!sq) return 0;
    g_last_error = "the poller's SG task-queue mode is switched off in this library: start() will refuse to run";
    return GFD_ERR_NOT_SUPPORTED;
}
int gfd_poller_start(gfd_poller_t p) {
    if (!p) return fail(1, "null poller");
    P(p)->start();
    if (P(p)->is_running()) return 0;
    g_last_error = "start(): the polling thread did not start (no descriptor queue, init_copy_engine() not done, "
                   "or an SG task queue is set)";
    return -1;
}
void gfd_poller_stop(gfd_poller_t p) {
    if (p) P(p)->stop();
}
int gfd_poller_is_running(gfd_poller_t p) { return p && P(p)->is_running() ? 1 : 0; }

int gfd_poller_get_stats(gfd_poller_t p, gfd_poller_stats* out) {
    if (!p || !out) return -1;
    auto* t = P(p);
    out->descriptors_processed = t->get_descriptors_processed();
    out->batches_submitted = t->get_batches_submitted();
    out->coalesced_entries = t->get_coalesced_entries();
    out->staging_batches = t->get_staging_batches();
    out->total_bytes_copied = t->get_total_bytes_copied();
    out->gather_us = t->get_gather_us();
    out->dma_wait_us = t->get_dma_wait_us();
    out->dma_submit_us = t->get_dma_submit_us();
    out->queue_read_us = t->get_queue_read_us();
    return 0;
}

void gfd_poller_reset_stats(gfd_poller_t p) {
    if (p) P(p)->reset_stats();
}

int gfd_poller_get_info(gfd_poller_t p, gfd_poller_info* out) {
    if (!p || !out) return -1;
    auto* t = P(p);
    std::memset(out, 0, sizeof(*out));
    out->device = t->device();
    out->numa_node = t->numa_node();
    out->num_gather_workers = t->num_gather_workers();
    out->poller_cpu = t->poller_cpu();
    const auto& w = t->worker_cpus();
    for (size_t i = 0; i < w.size() && i < 16; i++) out->worker_cpus[i] = w[i];
    out->num_ce_channels = t->get_ce_manager().num_channels();
    out->num_staging_buffers = t->num_staging_buffers();
    out->staging_buffer_size = t->staging_buffer_size();
    out->direct_chunk_bytes = t->direct_chunk_bytes();
    out->gather_slice_bytes = t->gather_slice_bytes();
    out->staging_pool_set = t->staging_pool_set();
    out->running = t->is_running() ? 1 : 0;
    return 0;
}

void gfd_poller_set_trace(gfd_poller_t p, int on) {
    if (p) P(p)->set_trace(on != 0);
}

int gfd_poller_read_trace(gfd_poller_t p, gfd_trace_event* out, int max) {
    static_assert(sizeof(gfd_trace_event) == sizeof(gfd::CpuPollingThread::TraceEvent), "trace event layout");
    if (!p || !out || max <= 0) return 0;
    return P(p)->read_trace(reinterpret_cast<gfd::CpuPollingThread::TraceEvent*>(out), max);
}

void gfd_poller_set_copy_timing(gfd_poller_t p, int on) {
    if (p) P(p)->set_copy_timing(on != 0);
}

int gfd_poller_read_copy_times(gfd_poller_t p, gfd_copy_time* out, int max) {
    static_assert(sizeof(gfd_copy_time) == sizeof(gfd::CpuPollingThread::CopyTiming), "copy time layout");
    if (!p || !out || max <= 0) return 0;
    return P(p)->read_copy_times(reinterpret_cast<gfd::CpuPollingThread::CopyTiming*>(out), max);
}

uint64_t gfd_poller_copy_clock_ns(gfd_poller_t p) { return p ? P(p)->copy_clock_ns() : 0; }

void gfd_poller_set_direct_zero_copy_max_bytes(gfd_poller_t p, uint64_t b) {
    if (p) P(p)->set_direct_zero_copy_max_bytes(b);
}
uint64_t gfd_poller_set_direct_zero_copy_min_bytes(gfd_poller_t p, uint64_t b) {
    if (!p) return 0;
    const uint64_t prev = P(p)->direct_zero_copy_min_bytes();
    P(p)->set_direct_zero_copy_min_bytes(b);
    return prev;
}
uint64_t gfd_poller_set_direct_zero_copy_head_bytes(gfd_poller_t p, uint64_t b) {
    if (!p) return 0;
    const uint64_t prev = P(p)->direct_zero_copy_head_bytes();
    P(p)->set_direct_zero_copy_head_bytes(b);
    return prev;
}
int gfd_poller_set_zero_copy_worker(gfd_poller_t p, int on) {
    if (!p) return fail(-1, "gfd_poller_set_zero_copy_worker: NULL poller");
    return P(p)->set_zero_copy_worker(on != 0) == 0
               ? 0
               : fail(-1, "gfd_poller_set_zero_copy_worker: set-up failed or the polling thread is running");
}
int gfd_poller_zero_copy_worker_stats(gfd_poller_t p, uint64_t* jobs, uint64_t* launches) {
    if (!p || !jobs || !launches) return fail(-1, "gfd_poller_zero_copy_worker_stats: invalid argument");
    *jobs = P(p)->zero_copy_worker_jobs();
    *launches = P(p)->zero_copy_worker_launches();
    return 0;
}
int gfd_poller_zero_copy_worker_timeline(gfd_poller_t p, uint64_t* out, int max_jobs) {
    if (!p || (!out && max_jobs > 0)) return 0;
    return P(p)->zero_copy_worker_timeline(out, max_jobs);
}
uint64_t gfd_poller_set_worker_queue_max_bytes(gfd_poller_t p, uint64_t b) {
    if (!p) return 0;
    const uint64_t prev = P(p)->worker_queue_max_bytes();
    P(p)->set_worker_queue_max_bytes(b);
    return prev;
}
void gfd_poller_set_direct_chunk_bytes(gfd_poller_t p, uint64_t b) {
    if (p) P(p)->set_direct_chunk_bytes(b);
}
void gfd_poller_set_gather_slice_bytes(gfd_poller_t p, uint64_t b) {
    if (p) P(p)->set_gather_slice_bytes(b);
}

namespace {
struct OrderCtx {
    int* order;
    int cap;
    int n;
};
void record_chunk(void* p, int chunk, size_t, size_t) {
    OrderCtx* c = (OrderCtx*)p;
    if (c->order && c->n < c->cap) c->order[c->n] = chunk;
    c->n++;
}

}  // namespace

int gfd_host_gather(const gfd_sg_entry* entries, int count, void* out, uint64_t chunk_bytes,
                    uint64_t slice_bytes, int num_workers, int* chunk_order, int chunk_order_cap) {
    if (count < 0 || (count > 0 && (!entries || !out)) || num_workers < 0 || num_workers > 64 ||
        chunk_order_cap < 0) {
        g_last_error = "gfd_host_gather: invalid argument";
        return -1;
    }
    if (count == 0) return 0;
    auto* e = reinterpret_cast<const gfd::SGEntry*>(entries);
    std::vector<int> cpus((size_t)num_workers, -1);
    gfd::GatherEngine engine(cpus);
    // The same list scan as submit_direct (parallel over the workers for long lists).
    const gfd::GatherEngine::ListScan sc = engine.scan(e, count);
    if (!sc.dst_contig) {
        g_last_error = "gfd_host_gather: destinations are not contiguous";
        return -1;
    }
    const size_t total = sc.total;
    if (slice_bytes) engine.set_slice_bytes(slice_bytes);
    OrderCtx ctx{chunk_order, chunk_order ? chunk_order_cap : 0, 0};
    engine.run(e, count, total, (char*)out, chunk_bytes, record_chunk, &ctx);
    return ctx.n;
}

int gfd_bench_host_gather(const gfd_sg_entry* const* lists, int nlists, int count, void* out,
                          uint64_t chunk_bytes, int num_workers, const int* cpus, int warmup, int iters,
                          double* times_us) {
    if (!lists || nlists <= 0 || count <= 0 || !out || num_workers < 0 || num_workers > 64 || !cpus ||
        warmup < 0 || iters <= 0 || !times_us) {
        g_last_error = "gfd_bench_host_gather: invalid argument";
        return -1;
    }
    for (int i = 0; i < nlists; i++)
        if (!lists[i]) {
            g_last_error = "gfd_bench_host_gather: null list";
            return -1;
        }
    std::vector<gfd::GatherEngine::ListScan> scans;
    std::vector<int> worker_cpus(cpus + 1, cpus + 1 + num_workers);
    gfd::GatherEngine engine(worker_cpus);
    for (int i = 0; i < nlists; i++) {
        scans.push_back(engine.scan(reinterpret_cast<const gfd::SGEntry*>(lists[i]), count));
        if (!scans.back().dst_contig) {
            g_last_error = "gfd_bench_host_gather: destinations are not contiguous";
            return -1;
        }
    }
    cpu_set_t saved;
    const bool have_saved = pthread_getaffinity_np(pthread_self(), sizeof(saved), &saved) == 0;
    if (cpus[0] >= 0) {
        cpu_set_t one;
        CPU_ZERO(&one);
        CPU_SET(cpus[0], &one);
        pthread_setaffinity_np(pthread_self(), sizeof(one), &one);
    }
    for (int it = -warmup; it < iters; it++) {
        const int k = (it + warmup) % nlists;
        const auto t0 = std::chrono::steady_clock::now();
        engine.run(reinterpret_cast<const gfd::SGEntry*>(lists[k]), count, scans[(size_t)k].total, (char*)out,
                   chunk_bytes, nullptr, nullptr);
        const auto t1 = std::chrono::steady_clock::now();
        if (it >= 0) times_us[it] = std::chrono::duration<double, std::micro>(t1 - t0).count();
    }
    if (have_saved) pthread_setaffinity_np(pthread_self(), sizeof(saved), &saved);
    return 0;
}

int gfd_staging_pool_init(int num_gpus, size_t buf_size, int numa_node) {
    return gfd::StagingPool::instance().init(num_gpus, buf_size, numa_node) ? 0 : -1;
}
void gfd_staging_pool_shutdown(void) { gfd::StagingPool::instance().shutdown(); }

// ---- measurement helpers ----

int gfd_bench_memcpy_per_token(void* dst, const uint64_t* src_addrs, int n, uint32_t T, int warmup, int iters,
                               double* times_us) {
    gfd_stream_t s = nullptr;
    CAPI_CHECK(gfd_hip_stream_create(&s), "hipStreamCreate");
    const uint64_t d0 = (uint64_t)(uintptr_t)dst;
    for (int it = -warmup; it < iters; it++) {
        auto t0 = std::chrono::steady_clock::now();
        for (int j = 0; j < n; j++) {
            int e = gfd_hip_memcpy_h2d_async(d0 + (uint64_t)j * T, (const void*)(uintptr_t)src_addrs[j], T, s);
            if (e) {
                gfd_hip_stream_destroy(s);
                return fail(e, "hipMemcpyAsync");
            }
        }
        int e = gfd_hip_stream_synchronize(s);
        auto t1 = std::chrono::steady_clock::now();
        if (e) {
            gfd_hip_stream_destroy(s);
            return fail(e, "hipStreamSynchronize");
        }
        if (it >= 0) times_us[it] = elapsed_us(t0, t1);
    }
    gfd_hip_stream_destroy(s);
    return 0;
}

int gfd_bench_memcpy_contiguous(void* dst, const void* src, size_t bytes, int ns, int warmup, int iters,
                                double* times_us) {
    if (ns < 1) ns = 1;
    if (ns > 8) ns = 8;
    gfd_stream_t st[8] = {};
    for (int i = 0; i < ns; i++) CAPI_CHECK(gfd_hip_stream_create(&st[i]), "hipStreamCreate");
    size_t per = ((bytes + ns - 1) / ns + 4095) & ~(size_t)4095;
    int rc = 0;
    for (int it = -warmup; it < iters && !rc; it++) {
        auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < ns && !rc; i++) {
            size_t off = (size_t)i * per;
            if (off >= bytes) break;
            size_t len = std::min(per, bytes - off);
            rc = gfd_hip_memcpy_h2d_async((uint64_t)(uintptr_t)dst + off, (const char*)src + off, len, st[i]);
        }
        for (int i = 0; i < ns && !rc; i++) rc = gfd_hip_stream_synchronize(st[i]);
        auto t1 = std::chrono::steady_clock::now();
        if (it >= 0) times_us[it] = elapsed_us(t0, t1);
    }
    for (int i = 0; i < ns; i++) gfd_hip_stream_destroy(st[i]);
    return rc ? fail(rc, "contiguous copy") : 0;
}

int gfd_bench_sdma_contiguous(void* dst, const void* src, size_t bytes, int channels, int pin, int warmup,
                              int iters, double* times_us, uint32_t* engine_mask) {
    int dev = 0;
    gfd_hip_get_device(&dev);
    gfd::SdmaQueue q;
    int st = q.init(dev, channels, pin);
    if (st) {
        g_last_error = "SDMA init failed";
        return st;
    }
    if (engine_mask) *engine_mask = q.engine_mask();
    if (channels < 1) channels = 1;
    const size_t per = ((bytes + channels - 1) / channels + 4095) & ~(size_t)4095;
    for (int it = -warmup; it < iters; it++) {
        auto t0 = std::chrono::steady_clock::now();
        for (int c = 0; c < channels; c++) {
            size_t off = (size_t)c * per;
            if (off >= bytes) break;
            size_t len = std::min(per, bytes - off);
            st = q.copy(c, (uint64_t)(uintptr_t)dst + off, (const char*)src + off, len);
            if (st) {
                q.wait_all();
                g_last_error = "SDMA copy failed";
                return st;
            }
        }
        if (q.wait_all()) {
            g_last_error = "SDMA copy reported an error";
            return -1;
        }
        auto t1 = std::chrono::steady_clock::now();
        if (it >= 0) times_us[it] = elapsed_us(t0, t1);
    }
    return 0;
}

int gfd_bench_submit_direct(gfd_poller_t p, const gfd_sg_entry* entries, int count, int warmup, int iters,
                            double* times_us) {
    if (!p) return -1;
    for (int it = -warmup; it < iters; it++) {
        double us = P(p)->submit_direct(reinterpret_cast<const gfd::SGEntry*>(entries), count);
        if (us < 0) {
            g_last_error = "submit_direct failed";
            return -1;
        }
        if (it >= 0) times_us[it] = us;
    }
    return 0;
}

int gfd_bench_zero_copy_scatter_tokens(const uint64_t* dst_addrs, const void* src, uint32_t T, int n, int warmup,
                                       int iters, double* wall_us, double* event_us) {
    return bench_kernel([&](gfd_stream_t s) { return gfd_zero_copy_scatter_tokens(dst_addrs, src, T, n, s); },
                        warmup, iters, wall_us, event_us, "zero-copy scatter");
}

int gfd_bench_memcpy_contiguous_d2h(void* dst, const void* src, size_t bytes, int ns, int warmup, int iters,
                                    double* times_us) {
    if (ns < 1) ns = 1;
    if (ns > 8) ns = 8;
    gfd_stream_t st[8] = {};
    for (int i = 0; i < ns; i++) CAPI_CHECK(gfd_hip_stream_create(&st[i]), "hipStreamCreate");
    const size_t per = ((bytes + ns - 1) / ns + 4095) & ~(size_t)4095;
    int rc = 0;
    for (int it = -warmup; it < iters && !rc; it++) {
        auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < ns && !rc; i++) {
            const size_t off = (size_t)i * per;
            if (off >= bytes) break;
            const size_t len = std::min(per, bytes - off);
            rc = gfd_hip_memcpy_d2h_async((char*)dst + off, (uint64_t)(uintptr_t)src + off, len, st[i]);
        }
        for (int i = 0; i < ns && !rc; i++) rc = gfd_hip_stream_synchronize(st[i]);
        auto t1 = std::chrono::steady_clock::now();
        if (it >= 0) times_us[it] = elapsed_us(t0, t1);
    }
    for (int i = 0; i < ns; i++) gfd_hip_stream_destroy(st[i]);
    return rc ? fail(rc, "contiguous D2H copy") : 0;
}

int gfd_bench_zero_copy_tokens_signal(const uint64_t* src_addrs, void* dst, uint32_t T, int n, int warmup,
                                      int iters, double* wall_us) {
    gfd_stream_t s = nullptr;
    void* counter = nullptr;
    uint64_t* word = nullptr;
    int rc = gfd_hip_stream_create(&s);
    if (!rc) rc = gfd_hip_malloc(&counter, 256);
    if (!rc) rc = gfd_hip_memset_d8((uint64_t)(uintptr_t)counter, 0, 256);
    if (!rc) rc = gfd_hip_device_synchronize();
    if (!rc) rc = gfd_hip_host_alloc((void**)&word, 64, GFD_HOST_COHERENT);
    if (!rc) *word = 0;
    for (int it = -warmup; it < iters && !rc; it++) {
        const uint64_t gen = (uint64_t)(it + warmup + 1);
        auto t0 = std::chrono::steady_clock::now();
        rc = gfd_zero_copy_gather_tokens_signal(src_addrs, dst, T, n, (unsigned int*)counter, word, gen, s);
        while (!rc && __atomic_load_n(word, __ATOMIC_ACQUIRE) != gen) {
            if (elapsed_us(t0, std::chrono::steady_clock::now()) > 10e6) {
                rc = gfd_hip_stream_synchronize(s);
                if (!rc && __atomic_load_n(word, __ATOMIC_ACQUIRE) != gen) rc = -1;
                break;
            }
        }
        auto t1 = std::chrono::steady_clock::now();
        if (it >= 0 && !rc) wall_us[it] = elapsed_us(t0, t1);
    }
    if (s) {
        gfd_hip_stream_synchronize(s);
        gfd_hip_stream_destroy(s);
    }
    if (counter) gfd_hip_free(counter);
    if (word) gfd_hip_host_free(word);
    return rc ? fail(rc, "zero-copy gather (signalled)") : 0;
}

int gfd_bench_zero_copy_tokens(const uint64_t* src_addrs, void* dst, uint32_t T, int n, int warmup, int iters,
                               double* wall_us, double* event_us) {
    return bench_kernel([&](gfd_stream_t s) { return gfd_zero_copy_gather_tokens(src_addrs, dst, T, n, s); },
                        warmup, iters, wall_us, event_us, "zero-copy gather");
}

int gfd_bench_queue(void* queue, const void* tokens, void* gpu_dst, int n, uint32_t T, uint64_t* base_slot,
                    int warmup, int iters, uint64_t timeout_us, double* times_us) {
    if (!queue || !base_slot) return -1;
    int* status = nullptr;
    CAPI_CHECK(gfd_hip_host_alloc((void**)&status, sizeof(int) * 16, GFD_HOST_COHERENT), "hipHostMalloc");
    gfd_stream_t s = nullptr;
    int rc = gfd_hip_stream_create(&s);
    for (int it = -warmup; it < iters && !rc; it++) {
        *status = -1;
        auto t0 = std::chrono::steady_clock::now();
        rc = gfd_queue_submit_tokens(queue, tokens, gpu_dst, n, T, *base_slot, s);
        if (rc) break;
        *base_slot += (uint64_t)n;
        rc = gfd_queue_wait(queue, *base_slot, timeout_us, status, s);
        if (!rc) rc = gfd_hip_stream_synchronize(s);
        auto t1 = std::chrono::steady_clock::now();
        if (!rc && __atomic_load_n(status, __ATOMIC_ACQUIRE) != 0) {
            g_last_error = "queue wait timed out";
            rc = -2;
        }
        if (it >= 0 && !rc) times_us[it] = elapsed_us(t0, t1);
    }
    if (s) gfd_hip_stream_destroy(s);
    gfd_hip_host_free(status);
    if (rc > 0) return fail(rc, "queue bench");
    return rc;
}

}  // extern "C"
