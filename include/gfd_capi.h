/*
 * gfd_capi.h — the C-ABI drop-in boundary of the MI355X GFD library
 * (libgfd_amd.so).  Plain pointers and sizes only; every function that can
 * fail returns 0 on success and a nonzero HIP/GFD error code otherwise
 * (gfd_last_error() gives a message for the calling thread).
 *
 * The C++ API in the include/gfd/ headers is the primary interface (same class names
 * and signatures as the reference's include/gfd).  These entry points wrap it
 * for FFI callers (ctypes, cgo, JNI) and are what the Python package binds.
 * Each declaration names the reference interface it replaces.
 */
#ifndef GFD_CAPI_H
#define GFD_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One host->device request; same 24-byte layout as gfd::SGEntry
 * (reference include/gfd/copy_engine.h:29-33: {CUdeviceptr dst; const void* src; size_t size}). */
typedef struct gfd_sg_entry {
    uint64_t dst;
    uint64_t src;
    uint64_t size;
} gfd_sg_entry;

typedef void* gfd_poller_t;

/* Counters of CpuPollingThread (reference include/gfd/cpu_polling.h:60-71). */
typedef struct gfd_poller_stats {
    uint64_t descriptors_processed;
    uint64_t batches_submitted;
    uint64_t coalesced_entries;
    uint64_t staging_batches;
    double total_bytes_copied;
    uint64_t gather_us;
    uint64_t dma_wait_us;
    uint64_t dma_submit_us;
    uint64_t queue_read_us;
} gfd_poller_stats;

/* Resources the poller chose (no reference counterpart; reported by the bench). */
typedef struct gfd_poller_info {
    int device;
    int numa_node;
    int num_gather_workers;
    int poller_cpu;
    int worker_cpus[16];
    int num_ce_channels;
    int num_staging_buffers;
    uint64_t staging_buffer_size;
    uint64_t direct_chunk_bytes;
    uint64_t gather_slice_bytes;
    int staging_pool_set;   /* StagingPool set of the Queue staging, -1 = self-allocated */
    int running;            /* polling thread running */
} gfd_poller_info;

/* Returned by entry points whose mode this library switches off. */
#define GFD_ERR_NOT_SUPPORTED 801
const char* gfd_version(void);
const char* gfd_last_error(void);

/* ---- runtime plumbing (the reference calls the CUDA runtime directly) ---- */
int gfd_device_count(int* n);
int gfd_set_device(int dev);
int gfd_device_synchronize(void);
/* flags: 0 default (pinned, coarse-grained), 1 coherent (fine-grained),
 * 2 non-coherent, 4 follow the thread's NUMA policy.
 * Replaces cudaHostAlloc / cudaMallocHost (examples/04_benchmark.cu:348). */
int gfd_host_alloc(void** p, size_t bytes, unsigned flags);
int gfd_host_free(void* p);
int gfd_device_alloc(void** p, size_t bytes);           /* cudaMalloc */
int gfd_device_free(void* p);
/* Blocking helpers: each returns once the operation is complete on the
 * device, so copies issued afterwards on other engines (SDMA, other streams)
 * cannot be overtaken by it. */
int gfd_memcpy_h2d(void* dst, const void* src, size_t n);
int gfd_memcpy_d2h(void* dst, const void* src, size_t n);
int gfd_memcpy_d2d(void* dst, const void* src, size_t n);
int gfd_memset_device(void* dst, int value, size_t n);
int gfd_stream_create(void** stream);                   /* non-blocking, default priority */
int gfd_stream_destroy(void* stream);
int gfd_stream_synchronize(void* stream);
int gfd_event_create(void** event);                     /* timing enabled */
int gfd_event_destroy(void* event);
int gfd_event_record(void* event, void* stream);
int gfd_event_synchronize(void* event);
int gfd_event_elapsed_ms(float* ms, void* start, void* stop);

/* ---- CpuPollingThread (reference include/gfd/cpu_polling.h:21-84) ---- */
/* CpuPollingThread::CpuPollingThread (cpu_polling.h:21-30); numa_node -1 = GPU-local. */
gfd_poller_t gfd_poller_create(void* queue, void* gpu_base, void* cpu_base, size_t total_cpu_size,
                               int use_ce, int numa_node, int core_offset, int num_ce_channels,
                               int exclusive_core_base, int exclusive_core_count);
void gfd_poller_destroy(gfd_poller_t p);                             /* ~CpuPollingThread */
int gfd_poller_init_copy_engine(gfd_poller_t p);                     /* init_copy_engine (:33) -> 0/err */
int gfd_poller_init_direct_ce(gfd_poller_t p);                       /* init_direct_ce (:43) */
/* submit_direct (cpu_polling.h:36-40, src/direct_submit.cpp:28): blocks until
 * the data is in HBM; returns elapsed microseconds, or -1 on error. */
double gfd_poller_submit_direct(gfd_poller_t p, const gfd_sg_entry* entries, int count);
void gfd_poller_set_tiled_queue(gfd_poller_t p, void* tiled_queue);  /* set_tiled_queue (:48) */
/* set_sg_task_queue (:53).  The poller's SG task-queue mode is switched off in
 * this library: the queue is recorded (start() then refuses to run) and the
 * call returns GFD_ERR_NOT_SUPPORTED with gfd_last_error() saying so. */
int gfd_poller_set_sg_task_queue(gfd_poller_t p, void* sg_queue);
/* start (:56).  0 once the polling thread runs; nonzero (and gfd_last_error())
 * if it did not start: no queue, init_copy_engine not done, or SG mode. */
int gfd_poller_start(gfd_poller_t p);
void gfd_poller_stop(gfd_poller_t p);                                /* stop (:57) */
int gfd_poller_is_running(gfd_poller_t p);                           /* 1 while the polling thread runs */
int gfd_poller_get_stats(gfd_poller_t p, gfd_poller_stats* out);     /* get_* (:60-71) */
void gfd_poller_reset_stats(gfd_poller_t p);                         /* reset_stats (:73) */
int gfd_poller_get_info(gfd_poller_t p, gfd_poller_info* out);
/* Timeline trace of the poller and direct path (no reference counterpart):
 * t_ns (CLOCK_MONOTONIC), kind (1 batch-first, 2 flush, 3 issued, 4 done,
 * 5 gap-flush, 6 direct-begin, 7 chunk, 8 direct-end, 9-13 gather job phases,
 * 14 zero-copy launch, 15 zero-copy completion seen), a, b as documented in
 * include/gfd/cpu_polling.h.  read_trace drains up to max events. */
typedef struct gfd_trace_event {
    uint64_t t_ns;
    uint32_t kind;
    uint32_t a;
    uint64_t b;
} gfd_trace_event;
void gfd_poller_set_trace(gfd_poller_t p, int on);
int gfd_poller_read_trace(gfd_poller_t p, gfd_trace_event* out, int max);
/* SDMA copy timeline (no reference counterpart; the reference times only
 * whole calls): engine start / end of every copy, in ns of the HSA system
 * clock, path 0 = Queue, 1 = Direct.  Enabling turns on the runtime's
 * async-copy profiling for the process. */
typedef struct gfd_copy_time {
    uint64_t seq, bytes, start_ns, end_ns;
    uint32_t channel, engine, path, _pad;
} gfd_copy_time;
void gfd_poller_set_copy_timing(gfd_poller_t p, int on);
int gfd_poller_read_copy_times(gfd_poller_t p, gfd_copy_time* out, int max);
uint64_t gfd_poller_copy_clock_ns(gfd_poller_t p);
/* Tuning of the pipelined direct path (no reference counterpart). */
void gfd_poller_set_direct_chunk_bytes(gfd_poller_t p, uint64_t bytes);
/* Destination-contiguous lists of at most `bytes` with pinned sources go
 * through the zero-copy kernel (0 = never). */
void gfd_poller_set_direct_zero_copy_max_bytes(gfd_poller_t p, uint64_t bytes);
/* Lists of at most `bytes` take the staged copy-engine route whatever the
 * maximum above (default 64 KiB: there a copy-engine copy completes sooner
 * than a kernel launch).  Returns the previous value. */
uint64_t gfd_poller_set_direct_zero_copy_min_bytes(gfd_poller_t p, uint64_t bytes);
/* Larger destination-contiguous lists with pinned sources: the zero-copy
 * kernel moves the first entries, up to `bytes`, while the rest is staged
 * for the copy engines (0 = staged only).  Returns the previous value. */
uint64_t gfd_poller_set_direct_zero_copy_head_bytes(gfd_poller_t p, uint64_t bytes);
/* The persistent zero-copy worker (no reference counterpart; it stands in for
 * the kernel launch and the copy-engine start of short copies,
 * CpuPollingThread::set_zero_copy_worker): on = 1 sets it up and routes
 * Direct lists of at most the zero-copy limit and Queue batches of at most
 * gfd_poller_set_worker_queue_max_bytes (4 MiB) with pinned sources through
 * it; 0 removes it.  Returns 0 or an error.  Not while the polling thread
 * runs. */
int gfd_poller_set_zero_copy_worker(gfd_poller_t p, int on);
/* Jobs posted to the worker and grids dispatched for them (both 0 while off). */
int gfd_poller_zero_copy_worker_stats(gfd_poller_t p, uint64_t* jobs, uint64_t* launches);
/* Returns the previous limit. */
uint64_t gfd_poller_set_worker_queue_max_bytes(gfd_poller_t p, uint64_t bytes);
/* The worker's device timeline of its latest jobs, newest first: up to
 * max_jobs records of 8 words on the GPU's 100 MHz wall clock (the last
 * workgroup to find the job, the last to hold it and its records, unused, the
 * last done copying, unused, the last progress word stored, the job number,
 * unused).  Returns the number of records (0 while the worker is off, or when
 * GFD_ZC_WORKER_TRACE=1 was not set as it started). */
int gfd_poller_zero_copy_worker_timeline(gfd_poller_t p, uint64_t* out, int max_jobs);
void gfd_poller_set_gather_slice_bytes(gfd_poller_t p, uint64_t bytes);

/* Host-only gather (no GPU): the staging step of the pipelined direct path.
 * Entries must have contiguous destinations; entry i lands at
 * out + (entries[i].dst - entries[0].dst).  chunk_order (optional) receives
 * the chunk indices in the order they were reported complete, at most
 * chunk_order_cap of them (every chunk but the last is at least
 * min(64 KiB, chunk_bytes) bytes, which bounds the count).  num_workers threads plus the caller.
 * Returns the number of chunks, or -1 on an invalid argument.  (Reference
 * counterpart: CpuPollingThread::parallel_gather, src/parallel_gather.cpp:74.) */
int gfd_host_gather(const gfd_sg_entry* entries, int count, void* out, uint64_t chunk_bytes,
                    uint64_t slice_bytes, int num_workers, int* chunk_order, int chunk_order_cap);

/* ---- StagingPool (reference include/gfd/staging_pool.h:50,176) ---- */
int gfd_staging_pool_init(int num_gpus, size_t buf_size, int numa_node);
void gfd_staging_pool_shutdown(void);

/* ---- zero-copy gather kernels (no reference counterpart: the GPU-initiated
 * form of the same gather contract) ---- */
/* dst + j*token_size <- src_addrs[j] (token_size bytes), j < num_tokens.
 * src_addrs: device-readable table (HBM or pinned host); tokens in pinned host memory. */
int gfd_zero_copy_gather_tokens(const uint64_t* src_addrs, void* dst, uint32_t token_size,
                                int num_tokens, void* stream);
/* Arbitrary SG list (device-readable array of entries, disjoint destinations).
 * Direction-agnostic: sources and destinations may each be HBM or pinned host
 * memory (H2D gather, D2H offload, D2D). */
int gfd_zero_copy_gather(const gfd_sg_entry* entries, int count, void* stream);
/* The same three kernels with completion signalled to the host instead of by
 * the stream (no reference counterpart; the reference waits on stream events):
 * when every byte has landed (and is visible to any agent), the grid's last
 * wave stores done_value to *done_word (pinned host memory, ideally coherent),
 * which the caller polls.  done_counter: one unsigned int in HBM, 0 before the
 * first launch; the kernel leaves it 0 again.  Launches that share a counter
 * must be ordered (one stream).  The stream still orders the launch as usual. */
int gfd_zero_copy_gather_tokens_signal(const uint64_t* src_addrs, void* dst, uint32_t token_size,
                                       int num_tokens, unsigned int* done_counter, uint64_t* done_word,
                                       uint64_t done_value, void* stream);
int gfd_zero_copy_scatter_tokens_signal(const uint64_t* dst_addrs, const void* src, uint32_t token_size,
                                        int num_tokens, unsigned int* done_counter, uint64_t* done_word,
                                        uint64_t done_value, void* stream);
int gfd_zero_copy_gather_signal(const gfd_sg_entry* entries, int count, unsigned int* done_counter,
                                uint64_t* done_word, uint64_t done_value, void* stream);
/* gfd_zero_copy_gather_signal for a table the caller has already cut into
 * pieces (no reference counterpart; used by submit_direct, whose
 * zc_fill_sg_table cuts a short list of large entries by size): the kernel
 * does not slice the entries again by count, so each record stays one wave's
 * work. */
int gfd_zero_copy_gather_signal_presliced(const gfd_sg_entry* entries, int count, unsigned int* done_counter,
                                          uint64_t* done_word, uint64_t done_value, void* stream);
/* Waves the zero-copy gather kernels give a short list (no reference
 * counterpart): GFD_ZC_WAVES when set, else 64.  A caller that cuts a list
 * into pieces for them sizes the pieces for this many waves. */
int gfd_zero_copy_target_waves(void);
/* GPU-built SG list for submit_direct (the pattern of examples/03_gpu_planned_transfer.cu:32-66,
 * plan_compact_kernel + plan_build_sg_kernel): the tokens t with routing[t] == expert, in token
 * order, become entries[k] = {gpu_dst + k*token_size, cpu_base + t*stride, token_size}, and
 * *count = their number.  routing: device-readable int[num_tokens]; entries and count may be
 * pinned host memory (the list is then ready for submit_direct once the stream is synchronised)
 * or HBM.  entries must hold every match.  Stable order, unlike the reference's atomicAdd slots. */
int gfd_plan_expert_entries(const int* routing, int num_tokens, int expert, const void* cpu_base,
                            uint64_t stride, void* gpu_dst, uint32_t token_size, gfd_sg_entry* entries,
                            int* count, void* stream);
/* Reverse path, no reference counterpart (the reference lists D2H as future
 * work, docs/Architecture.md:642,993): offload of KV pages from HBM to host.
 * dst_addrs[j] (pinned host) <- src + j*token_size (HBM), j < num_tokens.
 * dst_addrs: device-readable table (HBM or pinned host). */
int gfd_zero_copy_scatter_tokens(const uint64_t* dst_addrs, const void* src, uint32_t token_size,
                                 int num_tokens, void* stream);

/* ---- MoE-routed SG gather with a wave-specialised consumer (the SG
 * warp-specialised path, reference include/gfd/sg_warp_spec.cuh and
 * examples/09_sg_warp_spec.cu, kept entirely on the GPU) ---- */
/* Top-2 experts per token of logits[num_tokens][num_experts] (fp32, HBM;
 * ties -> lower expert id) into top2[2*num_tokens]; per-expert row lists in
 * token order: offsets[num_experts+1], row_token[2*num_tokens] (expert-major). */
int gfd_moe_route(const float* logits, int num_tokens, int num_experts, int* top2, int* offsets,
                  int* row_token, void* stream);
/* gfd_moe_route for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); no
 * counterpart in the reference.  The same offsets and row_token, with the
 * top-2 pairs kept in a scratch array the library holds in device memory
 * (one per GPU, 512 KiB, until the process ends) instead of a caller buffer.
 * Allocates nothing.  num_tokens <= 65536 (larger: an error, nothing launched).
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one
 * GPU (other streams or threads) race; calls ordered on one stream do not. */
int gfd_moe_route_noalloc(const float* logits, int num_tokens, int num_experts, int* offsets,
                          int* row_token, void* stream);
/* Row r: token row_token[r] (host_base + token*token_stride, row_bytes bytes,
 * pinned host memory) -> dst + r*row_bytes (HBM).  out != NULL: producer waves
 * fetch into an LDS ring and consumer waves write the bf16 RMSNorm
 * x / sqrt(mean(x^2) + eps) * weight to out + r*row_bytes; out == NULL: pure
 * transfer.  row_bytes a multiple of 1024, at most 14336.  num_blocks 0 =
 * min(CU count, 64) workgroups.  *error_flag (device int, zeroed by the
 * caller) receives nonzero bits on a bad token id or a stalled hand-off. */
int gfd_sg_gather_rmsnorm(const void* host_base, uint64_t token_stride, int num_tokens,
                          const int* row_token, int num_rows, uint32_t row_bytes, void* dst, void* out,
                          const uint16_t* weight, float eps, int num_blocks, int* error_flag, void* stream);

/* ---- GFD Queue mode (reference include/gfd/device.cuh, examples/04_benchmark.cu:31-54) ---- */
/* DescriptorQueue in fine-grained host memory, zeroed. */
int gfd_queue_alloc(void** queue);
int gfd_queue_free(void* queue);
/* bench_gfd_submit_kernel (examples/04_benchmark.cu:31-46): descriptor j =
 * {tokens[j].cpu_addr, gpu_dst + j*token_size, token_size, LAST_IN_BATCH on the last}
 * at slot base_slot + j, one wave64 lane per descriptor. */
int gfd_queue_submit_tokens(void* queue, const void* tokens, void* gpu_dst, int num_tokens,
                            uint32_t token_size, uint64_t base_slot, void* stream);
/* The same descriptors written with write_descriptor_safe (include/gfd/device.cuh:120-152):
 * each lane writes its slot only once the poller has consumed it, retrying (bounded by
 * timeout_us; then *status = 1).  num_tokens may exceed QUEUE_SIZE: later laps wait for the
 * ring.  full_count (HBM, optional) receives the number of lanes that found their slot full. */
int gfd_queue_submit_tokens_safe(void* queue, const void* tokens, void* gpu_dst, int num_tokens,
                                 uint32_t token_size, uint64_t base_slot, uint64_t timeout_us, int* status,
                                 unsigned int* full_count, void* stream);
/* bench_gfd_wait_kernel (examples/04_benchmark.cu:49-54) with a bound: spins
 * until done_idx >= expected_done or timeout_us elapses; *status (device or
 * host-visible int) receives 0 on completion, 1 on timeout. */
int gfd_queue_wait(void* queue, uint64_t expected_done, uint64_t timeout_us, int* status,
                   void* stream);
/* ---- the poller's tiled mode (TiledQueue, include/gfd/tiled_queue.h; reference
 * include/gfd/tiled_queue.h:8-43) driven by a kernel through include/gfd/device_primitives.h ---- */
/* TiledQueue in fine-grained host memory with its scheduler fields set; device_signals != 0
 * also allocates d_tile_chunk_done[MAX_TILES] in HBM (the poller then signals there with
 * copy-engine writes; otherwise it writes tile_chunk_done in host memory). */
int gfd_tiled_queue_alloc(void** tq, uint32_t total_tiles, uint32_t tokens_per_tile,
                          uint32_t tokens_per_chunk, uint32_t token_size, int device_signals);
int gfd_tiled_queue_free(void* tq);
/* Ring indices, sequences, progress words and next_tile back to zero (poller stopped). */
int gfd_tiled_queue_reset(void* tq);
/* baseline_kernel of examples/07_warp_spec_simple.cu:88-134: one workgroup per tile submits
 * its tokens (token g: cpu_base + g*T -> gpu_base + g*T) chunk by chunk (whole_tile: in one
 * go) and waits (bounded by timeout_us) for the tile's progress word; then sums[g] = the
 * u32-word checksum of token g as landed.  *status (0 from the caller) becomes 1 on a
 * timeout.  The whole launch must fit the ring (total_tiles * tokens_per_tile slots). */
int gfd_tiled_poller_run(void* tq, const void* cpu_base, void* gpu_base, int whole_tile,
                         uint64_t timeout_us, unsigned long long* sums, int* status, void* stream);
/* fused_prefetch_and_compute_kernel (examples/01_basic_transfer.cu:27-85) in one launch:
 * descriptors as gfd_queue_submit_tokens, then each workgroup waits (bounded by timeout_us)
 * until the poller has landed all num_tokens, then writes sums[j] = the u32-word checksum of
 * token j as landed in HBM (little-endian words, a trailing partial word byte by byte).
 * *status (set to 0 by the caller) becomes 1 if a wait timed out.  num_tokens <= QUEUE_SIZE. */
int gfd_queue_fused_checksums(void* queue, const void* tokens, void* gpu_dst, int num_tokens,
                              uint32_t token_size, uint64_t base_slot, uint64_t timeout_us,
                              unsigned long long* sums, int* status, void* stream);

/* ---- measurement helpers (examples/04_benchmark.cu:92-115 and the peak
 * reference copy); fill times_us[iters] with wall times ---- */
int gfd_bench_memcpy_per_token(void* dst, const uint64_t* src_addrs, int num_tokens,
                               uint32_t token_size, int warmup, int iters, double* times_us);
int gfd_bench_memcpy_contiguous(void* dst, const void* src, size_t bytes, int num_streams,
                                int warmup, int iters, double* times_us);
/* One contiguous copy split over `channels` SDMA channels (engines pinned when
 * pin != 0, else runtime-chosen); also reports the engine mask. */
int gfd_bench_sdma_contiguous(void* dst, const void* src, size_t bytes, int channels, int pin,
                              int warmup, int iters, double* times_us, uint32_t* engine_mask);
int gfd_bench_submit_direct(gfd_poller_t p, const gfd_sg_entry* entries, int count, int warmup,
                            int iters, double* times_us);
/* The product's host gather alone (the staging step of the Direct path,
 * reference counterpart CpuPollingThread::parallel_gather,
 * src/parallel_gather.cpp:74): one GatherEngine with num_workers threads
 * pinned to cpus[1..num_workers] and the caller pinned to cpus[0] for the
 * call (num_workers + 1 CPU ids), timing `iters` gathers after `warmup`;
 * gather k reads lists[k % nlists] (each `count` entries with contiguous
 * destinations, landing at out + (dst - lists[i][0].dst)), so several lists
 * over separate source regions give a cold source. */
int gfd_bench_host_gather(const gfd_sg_entry* const* lists, int nlists, int count, void* out,
                          uint64_t chunk_bytes, int num_workers, const int* cpus, int warmup, int iters,
                          double* times_us);
/* Zero-copy tokens kernel with its completion signalled to a host word:
 * wall time from the launch call until the host sees the word. */
int gfd_bench_zero_copy_tokens_signal(const uint64_t* src_addrs, void* dst, uint32_t token_size,
                                      int num_tokens, int warmup, int iters, double* wall_us);
/* Zero-copy tokens kernel: wall time launch->sync and HIP-event kernel time. */
int gfd_bench_zero_copy_tokens(const uint64_t* src_addrs, void* dst, uint32_t token_size,
                               int num_tokens, int warmup, int iters, double* wall_us,
                               double* event_us);
/* The same for the offload kernel (gfd_zero_copy_scatter_tokens). */
int gfd_bench_zero_copy_scatter_tokens(const uint64_t* dst_addrs, const void* src, uint32_t token_size,
                                       int num_tokens, int warmup, int iters, double* wall_us,
                                       double* event_us);
/* hipMemcpyAsync device->host of one contiguous range over num_streams
 * streams (the D2H link-rate reference). */
int gfd_bench_memcpy_contiguous_d2h(void* dst, const void* src, size_t bytes, int num_streams,
                                    int warmup, int iters, double* times_us);
/* Queue mode: submit kernel + wait kernel, wall time launch->device sync. */
int gfd_bench_queue(void* queue, const void* tokens, void* gpu_dst, int num_tokens,
                    uint32_t token_size, uint64_t* base_slot, int warmup, int iters,
                    uint64_t timeout_us, double* times_us);

/* ---- wave-specialised sessions (reference include/gfd/warp_spec_session.h,
 * src/warp_spec_session.cpp, src/sg_warp_spec_session.cpp).  The C++ classes
 * gfd::WarpSpecSession / gfd::SGWarpSpecSession are the primary API (kernels
 * are instantiated from user functors); these entry points drive them with
 * built-in consumers for FFI callers and tests. ---- */

/* Same 24-byte layout as gfd::DeviceSGEntry (reference include/gfd/sg_task_queue.h:37-43). */
typedef struct gfd_device_sg_entry {
    uint64_t src;
    uint64_t dst;
    uint32_t size;
    uint32_t tag;
} gfd_device_sg_entry;

/* get_stats() of a session (reference include/gfd/warp_spec_session.h:118-124)
 * plus what the kernels report. */
typedef struct gfd_session_result {
    uint64_t units_done;  /* tokens (WarpSpec) or entries (SG) landed: descriptors_processed */
    uint64_t bytes;       /* bytes_transferred */
    uint64_t lists_done;  /* tiles (WarpSpec) or lists (SG) landed */
    uint64_t error_bits;  /* nonzero: a bounded wait inside the kernel gave up */
    double elapsed_ms;    /* launch -> synchronize, host clock */
    int grid, block, tokens_per_chunk, chunks_per_tile;
    int helper_waves;     /* transfer helper waves per workgroup (an addition to the reference's API) */
} gfd_session_result;

/* WarpSpecSession over tokens [0, total_tokens) of cpu_src (pinned) -> gpu_dst
 * (HBM): construct, then `iters` times reset + launch + synchronize.
 * token_sums != NULL: the consumer writes each token's float sum to
 * token_sums[t] (test/test_db_small_tiles.cu:18-31); NULL: no-op consumer.
 * kernel_ms[iters] (optional) gets HIP-event times of each launch.
 * Tokens past the last whole tile are not moved (as the reference). */
/* helper_waves: transfer helper waves per workgroup (negative: about 32
 * transfer waves per launch, gfd::auto_helper_waves; fewer where the
 * workgroup would pass 1024 threads). */
int gfd_warp_spec_run(const void* cpu_src, void* gpu_dst, uint32_t total_tokens, uint32_t token_size,
                      uint32_t tokens_per_tile, uint32_t tokens_per_chunk, int double_buffer,
                      int per_tile_mode, int num_blocks, int helper_waves, float* token_sums, int iters,
                      double* kernel_ms, gfd_session_result* res);
/* The same run with the RMSNorm + sinf consumer of
 * examples/07_warp_spec_simple.cu:35-58 (VectorReduce): out[t] = sum over
 * token t's floats x of sin(x r) x r, r = 1 / sqrt(mean(x^2) + 1e-6), in
 * fp32 (device float[total_tokens]).  token_size a multiple of 4; chunk mode. */
int gfd_warp_spec_run_rms_sin(const void* cpu_src, void* gpu_dst, uint32_t total_tokens, uint32_t token_size,
                              uint32_t tokens_per_tile, uint32_t tokens_per_chunk, int double_buffer, int num_blocks,
                              int helper_waves, float* out, int iters, double* kernel_ms, gfd_session_result* res);

typedef void* gfd_sg_session_t;
/* SGWarpSpecSession(SGWarpSpecConfig{num_compute_warps, num_blocks}); idle_limit_ms
 * bounds how long transfer waves wait without a list (0 = 30 s); helper_waves
 * = transfer helper waves per workgroup, 0..3 (negative: about 32 transfer
 * waves per launch, gfd::auto_helper_waves). */
int gfd_sg_session_create(int num_compute_warps, int num_blocks, uint32_t idle_limit_ms, int helper_waves,
                          gfd_sg_session_t* out);
void gfd_sg_session_destroy(gfd_sg_session_t s);
/* submit_sg_list (warp_spec_session.h:170-171): returns the ring index, or -1. */
int64_t gfd_sg_session_submit(gfd_sg_session_t s, const gfd_device_sg_entry* entries, uint32_t count,
                              uint32_t list_id, uint32_t flags);
/* launch with the checksum consumer: list_sums[list_id] (device u64[512],
 * zeroed by the caller) += sum of the list's landed bytes as LE u32 words
 * (a trailing partial word adds its bytes); list_sums == NULL: no-op consumer
 * (test/test_sg_e2e.cu:10-17). */
int gfd_sg_session_launch(gfd_sg_session_t s, unsigned long long* list_sums, void* stream);
/* launch with the MoE consumer of examples/09_sg_warp_spec.cu:44-65: for entry i
 * of list list_id, out[list_id * count + i] = L2 norm of the landed bytes read
 * as fp32 (device float[out_len]; entries with an unaligned destination or a
 * slot past out_len are skipped). */
int gfd_sg_session_launch_l2norm(gfd_sg_session_t s, float* out, uint32_t out_len, void* stream);
/* Kernel with a submitter wave per workgroup (test/test_sg_gpu_submit.cu:20-213):
 * list i = entries [i*entries_per_list, (i+1)*entries_per_list) of d_entries
 * (device array), list_id i; the submitters set terminate once all landed. */
int gfd_sg_session_launch_gpu_submit(gfd_sg_session_t s, const gfd_device_sg_entry* d_entries,
                                     uint32_t entries_per_list, uint32_t num_lists,
                                     unsigned long long* list_sums, void* stream);
/* synchronize (sg_warp_spec_session.cpp:118-139): waits for every host-submitted
 * list and `extra_gpu_lists` GPU-submitted lists to land, sets terminate,
 * waits for the kernel.  Nonzero if lists did not land or the kernel
 * reported an error. */
/* The MoE-routed gather through the session (the SG MoE workload of
 * examples/09_sg_warp_spec.cu:78-294 with lists built on the GPU): submitter
 * waves cut expert e's rows [offsets[e], offsets[e+1]) of gfd_moe_route's
 * expert-major order into lists of at most rows_per_list (1..64) rows (list
 * ids 0..: every expert's full lists in expert order, then the shorter
 * remainder lists, longest first); entry r: src = host_base +
 * row_token[r] * token_stride (pinned host), dst = dst + r * row_bytes (HBM),
 * tag = r.  The transfer waves copy each list; with out != NULL the compute
 * wave writes the bf16 RMSNorm x / sqrt(mean(x^2) + eps) * weight of every
 * landed row to out + r * row_bytes (row_bytes a multiple of 1024, at most
 * 14 KiB), else it does nothing.  offsets / row_token / weight are
 * device-readable; at most 64 experts and MAX_SG_POOL_ENTRIES rows (lists
 * beyond MAX_SG_LISTS reuse ring slots; their ids get no d_list_done word).  The kernel ends
 * itself once every list has landed: synchronise the stream, then call
 * gfd_sg_session_synchronize(s, 0).  Routing entries out of range are
 * skipped and reported as error bit 16. */
int gfd_sg_session_launch_moe(gfd_sg_session_t s, const void* host_base, uint64_t token_stride, int num_tokens,
                              const int* offsets, const int* row_token, int num_experts, int num_rows,
                              uint32_t row_bytes, uint32_t rows_per_list, void* dst, void* out,
                              const uint16_t* weight, float eps, void* stream);
int gfd_sg_session_synchronize(gfd_sg_session_t s, uint64_t extra_gpu_lists);
int gfd_sg_session_reset(gfd_sg_session_t s);
int gfd_sg_session_stats(gfd_sg_session_t s, gfd_session_result* out);
void* gfd_sg_session_queue(gfd_sg_session_t s); /* get_sg_queue(): the SGTaskQueue */
/* Per-list device timeline of the session's launches; no counterpart in the
 * reference.  From the next launch on, the transfer waves record each of the
 * launch's first max_lists lists, in ring order, and each workgroup
 * (max_lists 0 switches it off).  Times are ticks of the device's 100 MHz
 * wall clock: claimed = the transfer wave starts looking for the list, ready =
 * its header is read and the copy starts, landed = its bytes are released
 * device-wide.  A list record still all 0 was not claimed. */
typedef struct {
    uint64_t claimed, ready, landed;
    uint32_t block, list_id;
} gfd_sg_trace_list;
/* start / exit of the workgroup's transfer wave, lists it copied */
typedef struct {
    uint64_t start, exit, lists, _pad;
} gfd_sg_trace_block;
int gfd_sg_session_enable_trace(gfd_sg_session_t s, uint32_t max_lists);
/* The last launch's records, after gfd_sg_session_synchronize: up to
 * max_lists / max_blocks records; their counts in *n_lists / *n_blocks. */
int gfd_sg_session_read_trace(gfd_sg_session_t s, gfd_sg_trace_list* lists, uint32_t max_lists,
                              gfd_sg_trace_block* blocks, uint32_t max_blocks, uint32_t* n_lists,
                              uint32_t* n_blocks);
/* Host-submitted SG transfer (`count` entries in lists of entries_per_list,
 * at most 16384 entries / 512 lists), no-op consumer: wall time from launch
 * until every list's done marker is up, times_us[iters]. */
int gfd_bench_sg_session(gfd_sg_session_t s, const gfd_device_sg_entry* entries, uint32_t count,
                         uint32_t entries_per_list, int warmup, int iters, double* times_us);

/* ---- the poller's SG mode (set_sg_task_queue; reference src/batch_processor.cpp:307-446)
 * driven by a kernel with the reference's SG transfer-warp protocol
 * (include/gfd/sg_warp_spec.cuh:95-262).  Switched off in this library:
 * gfd_poller_start refuses a poller with an SG task queue set, because runs of
 * the mode aborted the process on MI355X and the cause is not found.  GPU-built
 * SG lists run through the gfd_sg_session_* entry points instead. ---- */
/* SGTaskQueue in fine-grained host memory; d_list_done (MAX_SG_LISTS flags + device counters)
 * in HBM when device_flags != 0 (the poller writes the flags with copy-engine writes after
 * each list's copies), else in fine-grained host memory (host stores at completion). */
int gfd_sg_task_queue_alloc(void** sg_queue, int device_flags);
int gfd_sg_task_queue_free(void* sg_queue);
int gfd_sg_task_queue_reset(void* sg_queue);  /* flags and lists_completed back to zero */
/* Workgroup l posts list l = d_entries[d_list_offsets[l] .. d_list_offsets[l+1]) as descriptors
 * (user_data = l << 32 | i, FLAG_LAST_IN_TILE on the last entry) into `queue`, waits (bounded
 * by timeout_us) for d_list_done[l], then adds the u32-word checksum of every landed entry to
 * list_sums[l] (zeroed by the caller).  *status (0 from the caller) becomes 1 on a timeout.
 * num_lists <= MAX_SG_LISTS; total_entries (the sum of the list sizes) must fit the ring.
 * Currently switched off (returns hipErrorNotSupported): its first GPU run aborted and the
 * cause is not yet known. */
int gfd_sg_poller_run(void* queue, void* sg_queue, const gfd_device_sg_entry* d_entries,
                      const uint32_t* d_list_offsets, int num_lists, uint32_t total_entries,
                      uint64_t timeout_us, unsigned long long* list_sums, int* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GFD_CAPI_H */
