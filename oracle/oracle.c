/*
 * oracle.c — CPU oracle for the scattered host-to-device gather path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file verifies results: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * product library (gfd_amd/libgfd_amd.so) never links or calls it.
 *
 * Contents and what each one restates:
 *   xorshift64 / fill / permutation  — the synthetic-layout generators (seeded
 *       xorshift64, Marsaglia 2003, shifts 13/7/17; Fisher–Yates from i=n-1
 *       down with j = next % (i+1)).  The reference has no generator of its
 *       own (its benchmark fills 0xAB, examples/04_benchmark.cu:350); these
 *       are pinned by Marsaglia's published sequence and by brute force.
 *   oracle_expected_gather — the closed form of the reference gather for a
 *       contiguous destination: out[e.dst - min_dst + b] = e.src[b]
 *       (src/parallel_gather.cpp:61-64, :105-106).
 *   oracle_pool_* — a restatement of CpuPollingThread::parallel_gather and
 *       gather_worker_loop (src/parallel_gather.cpp:44-116): W spinning worker
 *       threads plus the caller, ceil(count/(W+1)) contiguous entry ranges,
 *       caller takes range 0, 16-entry software prefetch, 64-byte
 *       unaligned-load + non-temporal-store copy with a memcpy tail and a
 *       store fence (src/parallel_gather.cpp:10-27).  It is the CPU baseline
 *       ("kind": "port") and a second, independently written gather that the
 *       closed form is checked against.
 *   oracle_expected_scatter — the offload (HBM -> host) closed form, the
 *       inverse of oracle_expected_gather; no reference counterpart.
 *   oracle_fnv1a64 — FNV-1a 64-bit hash used by the golden fixtures.
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <immintrin.h>

#define ORACLE_API __attribute__((visibility("default")))

/* Same 24-byte layout as gfd::SGEntry (include/gfd/copy_engine.h:29-33). */
typedef struct {
    uint64_t dst;
    const void* src;
    size_t size;
} oracle_sg_entry;

/* ---------------------------------------------------------------- RNG */

ORACLE_API uint64_t oracle_xorshift64_next(uint64_t* state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

ORACLE_API void oracle_xorshift64_fill(uint64_t seed, uint64_t* out, size_t n) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) out[i] = oracle_xorshift64_next(&s);
}

/*
 * Fill a source region with num_tokens tokens of token_size bytes placed at
 * `stride` bytes apart.  Token bytes are the little-endian byte stream of
 * successive xorshift64 outputs: token k holds stream bytes
 * [k*token_size, (k+1)*token_size).  Every byte outside the tokens is `gap`.
 */
ORACLE_API void oracle_fill_tokens(uint8_t* region, size_t num_tokens, size_t token_size,
                                   size_t stride, uint64_t seed, uint8_t gap) {
    uint64_t s = seed;
    uint64_t word = 0;
    int avail = 0;
    for (size_t k = 0; k < num_tokens; k++) {
        uint8_t* t = region + k * stride;
        size_t b = 0;
        /* fast path: whole words when aligned in the stream */
        while (b < token_size) {
            if (avail == 0 && token_size - b >= 8) {
                uint64_t w = oracle_xorshift64_next(&s);
                memcpy(t + b, &w, 8); /* little-endian host */
                b += 8;
                continue;
            }
            if (avail == 0) {
                word = oracle_xorshift64_next(&s);
                avail = 8;
            }
            t[b++] = (uint8_t)(word & 0xFF);
            word >>= 8;
            avail--;
        }
        if (stride > token_size) memset(t + token_size, gap, stride - token_size);
    }
}

/* Fisher–Yates, i = n-1 .. 1, j = next % (i+1). */
ORACLE_API void oracle_permutation(uint32_t* perm, size_t n, uint64_t seed) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) perm[i] = (uint32_t)i;
    if (n < 2) return;
    for (size_t i = n - 1; i >= 1; i--) {
        size_t j = (size_t)(oracle_xorshift64_next(&s) % (uint64_t)(i + 1));
        uint32_t t = perm[i];
        perm[i] = perm[j];
        perm[j] = t;
    }
}

/* ------------------------------------------------------ closed form */

/*
 * Closed form for the benchmark layout: entry j reads token perm[j] at
 * region + perm[j]*stride and lands at out + j*token_size.
 */
ORACLE_API void oracle_expected_gather(uint8_t* out, const uint8_t* region, const uint32_t* perm,
                                       size_t n, size_t token_size, size_t stride) {
    for (size_t j = 0; j < n; j++)
        memcpy(out + j * token_size, region + (size_t)perm[j] * stride, token_size);
}

/*
 * Closed form for an arbitrary SG list with disjoint destinations:
 * out[e.dst - min_dst + b] = e.src[b]  (src/parallel_gather.cpp:61-64).
 */
ORACLE_API void oracle_gather_entries(uint8_t* out, const oracle_sg_entry* e, int count,
                                      uint64_t min_dst) {
    for (int i = 0; i < count; i++) {
        const uint8_t* s = (const uint8_t*)e[i].src;
        uint8_t* d = out + (e[i].dst - min_dst);
        for (size_t b = 0; b < e[i].size; b++) d[b] = s[b];
    }
}

/*
 * Offload (reverse path, no reference counterpart: the reference lists D2H
 * as future work, docs/Architecture.md:642,993): token j of a contiguous
 * device range, tokens + j*token_size, lands at region + perm[j]*stride.
 * Bytes of `region` no token covers keep their value.  It is the inverse of
 * oracle_expected_gather on the tokens' bytes.
 */
ORACLE_API void oracle_expected_scatter(uint8_t* region, const uint8_t* tokens, const uint32_t* perm,
                                        size_t n, size_t token_size, size_t stride) {
    for (size_t j = 0; j < n; j++)
        memcpy(region + (size_t)perm[j] * stride, tokens + j * token_size, token_size);
}

ORACLE_API uint64_t oracle_fnv1a64(const uint8_t* p, size_t n) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (size_t i = 0; i < n; i++) {
        h ^= p[i];
        h *= 0x100000001b3ULL;
    }
    return h;
}

/* --------------------------------------- parallel gather restatement */

/* 64-byte unaligned load + non-temporal store, memcpy tail, store fence
 * (src/parallel_gather.cpp:10-27).  AVX-512 when the CPU has it, else AVX2
 * (two 32-byte halves) — the destination of a streaming store must be
 * aligned, so misaligned destinations take the memcpy path. */
__attribute__((target("avx512f"))) static void stream_copy_avx512(uint8_t* d, const uint8_t* s,
                                                                   size_t n) {
    size_t aligned = n & ~(size_t)63;
    for (size_t i = 0; i < aligned; i += 64) {
        __m512i v = _mm512_loadu_si512((const void*)(s + i));
        _mm512_stream_si512((void*)(d + i), v);
    }
    if (aligned < n) memcpy(d + aligned, s + aligned, n - aligned);
    _mm_sfence();
}

__attribute__((target("avx2"))) static void stream_copy_avx2(uint8_t* d, const uint8_t* s,
                                                              size_t n) {
    size_t aligned = n & ~(size_t)63;
    for (size_t i = 0; i < aligned; i += 64) {
        __m256i a = _mm256_loadu_si256((const __m256i*)(s + i));
        __m256i b = _mm256_loadu_si256((const __m256i*)(s + i + 32));
        _mm256_stream_si256((__m256i*)(d + i), a);
        _mm256_stream_si256((__m256i*)(d + i + 32), b);
    }
    if (aligned < n) memcpy(d + aligned, s + aligned, n - aligned);
    _mm_sfence();
}

static int g_has_avx512 = -1;

static void stream_copy(uint8_t* d, const uint8_t* s, size_t n) {
    if (((uintptr_t)d & 63) != 0) {
        memcpy(d, s, n);
        return;
    }
    if (g_has_avx512 < 0) g_has_avx512 = __builtin_cpu_supports("avx512f") ? 1 : 0;
    if (g_has_avx512)
        stream_copy_avx512(d, s, n);
    else
        stream_copy_avx2(d, s, n);
}

static void copy_range(const oracle_sg_entry* e, int start, int end, uint8_t* staging,
                       uint64_t min_dst) {
    const int PF = 16; /* src/parallel_gather.cpp:50,93 */
    for (int p = 0; p < PF && start + p < end; p++) __builtin_prefetch(e[start + p].src, 0, 0);
    for (int i = start; i < end; i++) {
        if (i + PF < end) {
            __builtin_prefetch(e[i + PF].src, 0, 0);
            __builtin_prefetch(&e[i + PF], 0, 3);
        }
        stream_copy(staging + (e[i].dst - min_dst), (const uint8_t*)e[i].src, e[i].size);
    }
}

typedef struct {
    _Alignas(64) atomic_int has_work;
    _Alignas(64) atomic_int done;
    const oracle_sg_entry* entries;
    uint8_t* staging;
    uint64_t min_dst;
    int start, end;
    char pad[64];
} oracle_task;

typedef struct {
    int num_workers;
    atomic_int running;
    oracle_task* tasks;
    pthread_t* threads;
} oracle_pool;

typedef struct {
    oracle_pool* pool;
    int id;
} worker_arg;

static void* worker_main(void* p) {
    worker_arg* a = (worker_arg*)p;
    oracle_task* t = &a->pool->tasks[a->id];
    oracle_pool* pool = a->pool;
    free(a);
    while (atomic_load_explicit(&pool->running, memory_order_acquire)) {
        if (atomic_load_explicit(&t->has_work, memory_order_acquire)) {
            copy_range(t->entries, t->start, t->end, t->staging, t->min_dst);
            /* Clear has_work BEFORE raising done.  The reference stores done
             * first (src/parallel_gather.cpp:66-67); a caller that sees done
             * can then publish the next task before the late has_work = false
             * lands, and that store erases the new task (the caller waits
             * forever).  Output bytes are unaffected by the order. */
            atomic_store_explicit(&t->has_work, 0, memory_order_release);
            atomic_store_explicit(&t->done, 1, memory_order_release);
        } else {
            _mm_pause();
        }
    }
    return NULL;
}

/* cpus: optional list of num_workers+1 CPU ids (entry 0 is the caller's). */
ORACLE_API void* oracle_pool_create(int num_workers, const int* cpus) {
    oracle_pool* pool = (oracle_pool*)calloc(1, sizeof(oracle_pool));
    pool->num_workers = num_workers;
    atomic_store(&pool->running, 1);
    if (num_workers > 0) {
        if (posix_memalign((void**)&pool->tasks, 128, sizeof(oracle_task) * num_workers) != 0) {
            free(pool);
            return NULL;
        }
        memset(pool->tasks, 0, sizeof(oracle_task) * num_workers);
        pool->threads = (pthread_t*)calloc(num_workers, sizeof(pthread_t));
    }
    for (int w = 0; w < num_workers; w++) {
        worker_arg* a = (worker_arg*)malloc(sizeof(worker_arg));
        a->pool = pool;
        a->id = w;
        pthread_create(&pool->threads[w], NULL, worker_main, a);
        if (cpus) {
            cpu_set_t cs;
            CPU_ZERO(&cs);
            CPU_SET(cpus[w + 1], &cs);
            pthread_setaffinity_np(pool->threads[w], sizeof(cs), &cs);
        }
    }
    if (cpus) {
        cpu_set_t cs;
        CPU_ZERO(&cs);
        CPU_SET(cpus[0], &cs);
        sched_setaffinity(0, sizeof(cs), &cs);
    }
    return pool;
}

ORACLE_API void oracle_pool_destroy(void* p) {
    oracle_pool* pool = (oracle_pool*)p;
    if (!pool) return;
    atomic_store_explicit(&pool->running, 0, memory_order_release);
    for (int w = 0; w < pool->num_workers; w++) pthread_join(pool->threads[w], NULL);
    free(pool->threads);
    free(pool->tasks);
    free(pool);
}

/*
 * One parallel gather: ceil(count/(W+1)) entries per thread, workers take
 * ranges 1..W, the caller range 0, then spin-join
 * (src/parallel_gather.cpp:74-116).
 */
ORACLE_API void oracle_pool_gather(void* p, const oracle_sg_entry* entries, int count,
                                   uint8_t* staging, uint64_t min_dst) {
    oracle_pool* pool = (oracle_pool*)p;
    int nw = pool->num_workers;
    int chunk = (count + nw) / (nw + 1);
    for (int w = 0; w < nw; w++) {
        int start = (w + 1) * chunk;
        if (start >= count) continue;
        int end = start + chunk < count ? start + chunk : count;
        oracle_task* t = &pool->tasks[w];
        t->entries = entries;
        t->staging = staging;
        t->min_dst = min_dst;
        t->start = start;
        t->end = end;
        atomic_store_explicit(&t->done, 0, memory_order_release);
        atomic_store_explicit(&t->has_work, 1, memory_order_release);
    }
    copy_range(entries, 0, chunk < count ? chunk : count, staging, min_dst);
    for (int w = 0; w < nw; w++) {
        if ((w + 1) * chunk >= count) continue;
        while (!atomic_load_explicit(&pool->tasks[w].done, memory_order_acquire)) _mm_pause();
    }
}

/* Run `iters` gathers and write each one's wall time (µs) into times_us. */
ORACLE_API void oracle_pool_time(void* p, const oracle_sg_entry* entries, int count,
                                 uint8_t* staging, uint64_t min_dst, int iters, double* times_us) {
    for (int i = 0; i < iters; i++) {
        struct timespec t0, t1;
        clock_gettime(CLOCK_MONOTONIC, &t0);
        oracle_pool_gather(p, entries, count, staging, min_dst);
        clock_gettime(CLOCK_MONOTONIC, &t1);
        times_us[i] = (t1.tv_sec - t0.tv_sec) * 1e6 + (t1.tv_nsec - t0.tv_nsec) * 1e-3;
    }
}

ORACLE_API int oracle_has_avx512(void) { return __builtin_cpu_supports("avx512f") ? 1 : 0; }
