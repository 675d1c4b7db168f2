// Kernels and C-ABI entry points for the WarpSpec / SG-WarpSpec sessions.
//
// The device frameworks (include/gfd/warp_spec.h, sg_warp_spec.h) are
// header-only templates a user instantiates with their own functor, exactly as
// with the reference's GFD_WARP_SPEC_KERNEL / GFD_SG_WARP_SPEC_KERNEL.  This
// file instantiates them with the functors the reference's own tests use
// (per-token float sums: test/test_db_small_tiles.cu:18-31; a no-op consumer:
// test/test_sg_e2e.cu:10-17; a GPU submitter wave:
// test/test_sg_gpu_submit.cu:20-213) plus a per-list checksum consumer, so
// FFI callers and the tests can drive the sessions end to end.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <vector>

#include "gfd/sg_device_primitives.h"
#include "gfd/sg_warp_spec.h"
#include "gfd/warp_spec.h"
#include "gfd/warp_spec_session.h"
#include "capi_error.h"
#include "gfd_capi.h"

static_assert(sizeof(gfd_device_sg_entry) == sizeof(gfd::DeviceSGEntry), "gfd_device_sg_entry layout");
static_assert(sizeof(gfd_session_result) % 8 == 0, "gfd_session_result layout");

namespace {

using gfd::sg_warp_spec::SGListView;
using gfd::warp_spec::ChunkView;

// Wave sum of a float; every lane gets the result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ uint64_t wave_sum(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, 64);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, 64);
        v += ((uint64_t)hi << 32) | lo;
    }
    return v;
}

// out[global token] = sum of the token's floats (test_db_small_tiles.cu:18-31),
// summed by the whole wave with 16-byte loads from HBM.
struct TokenSum {
    float* out;
    __device__ void operator()(ChunkView c) const {
        const uint32_t nf = c.token_size / 4;
        for (uint32_t i = 0; i < c.size; i++) {
            const float* t = c.data<float>((int)i);
            float s = 0.f;
            for (uint32_t k = (uint32_t)c.lane_id; k < nf; k += 64) s += t[k];
            s = wave_sum(s);
            if (c.lane_id == 0) out[c.global_idx((int)i)] = s;
        }
    }
};

// out[global token] = sum over the token's floats x of sin(x r) x r, with
// r = 1 / sqrt(mean(x^2) + 1e-6): the RMSNorm + sinf consumer of
// examples/07_warp_spec_simple.cu:35-58 (VectorReduce).  There one lane
// walks a whole token twice; here the wave shares each token.
// One wave computes a whole chunk, so the last chunk of a launch is a tail
// no transfer overlaps.  For tokens of at most 16 KiB with 16-byte aligned
// floats the sum of squares issues all of a lane's (up to 16) 16-byte loads
// at once, so the wave waits on HBM once per token instead of once per 1 KiB;
// the sinf pass then reads the token again (from L2) two vectors at a time,
// which keeps the unrolled sinf code within the kernel's registers.  Lanes
// past the token read zeros, which add nothing to either sum
// (sin(0) * 0 = 0).  Other tokens take two lane-strided passes.  At 8192 x
// 16 KiB with 128-token tiles of 32-token chunks this took the kernel from
// 2761 to 2630 us.
template <bool kWholeToken>
struct TokenRmsSinT {
    float* out;
    static constexpr int kRegVecs = 16;  // float4 per lane: 16 KiB per wave
    // Each token's result depends on that token alone: the framework may
    // hand a chunk's tokens to several compute waves in groups.
    static constexpr bool kSplitsChunks = true;

    __device__ void operator()(ChunkView c) const {
        const uint32_t nf = c.token_size / 4;
        const uint32_t lane = (uint32_t)c.lane_id;
        if (((uintptr_t)c.base_ptr & 15) == 0 && (c.token_size & 15) == 0 && nf >= 4 && nf / 4 <= 64u * kRegVecs) {
            const uint32_t nv = nf / 4;
            if constexpr (kWholeToken) {
                // A kernel with room for 64 more registers per lane reads the
                // whole token at once for the sum of squares: one round trip
                // to HBM per token instead of four.  (The sinf pass then reads
                // the token again from L2 in batches: its unrolled code is too
                // large to keep the token in registers through it.)  A native
                // vector type: an array of 16 of HIP's float4 wrappers would
                // be placed in scratch memory.
                typedef float f4 __attribute__((ext_vector_type(4)));
                for (uint32_t i = 0; i < c.size; i++) {
                    const f4* t4 = c.data<f4>((int)i);
                    f4 x[kRegVecs];
#pragma unroll
                    for (int j = 0; j < kRegVecs; j++) {
                        const uint32_t k = lane + 64u * (uint32_t)j;
                        x[j] = t4[k < nv ? k : nv - 1];
                    }
                    float ss = 0.f;
#pragma unroll
                    for (int j = 0; j < kRegVecs; j++)
                        if (lane + 64u * (uint32_t)j < nv)
                            ss += x[j].x * x[j].x + x[j].y * x[j].y + x[j].z * x[j].z + x[j].w * x[j].w;
                    const float r = rsqrtf(wave_sum(ss) / (float)nf + 1e-6f);
                    const float4* v4 = c.data<float4>((int)i);
                    float acc = 0.f;
                    constexpr int kBatch = 4;
#pragma unroll
                    for (int j0 = 0; j0 < kRegVecs; j0 += kBatch) {
                        float4 y[kBatch];
#pragma unroll
                        for (int j = 0; j < kBatch; j++) {
                            const uint32_t k = lane + 64u * (uint32_t)(j0 + j);
                            y[j] = v4[k < nv ? k : nv - 1];
                        }
#pragma unroll
                        for (int j = 0; j < kBatch; j++) {
                            if (lane + 64u * (uint32_t)(j0 + j) >= nv) continue;
                            const float a = y[j].x * r, b = y[j].y * r, d = y[j].z * r, e = y[j].w * r;
                            acc += sinf(a) * a + sinf(b) * b + sinf(d) * d + sinf(e) * e;
                        }
                    }
                    acc = wave_sum(acc);
                    if (lane == 0) out[c.global_idx((int)i)] = acc;
                }
                return;
            }
            for (uint32_t i = 0; i < c.size; i++) {
                const float4* t4 = c.data<float4>((int)i);
                // Each pass reads the token in batches of kBatch vectors per
                // lane, every load of a batch issued before the first is used:
                // the index is clamped instead of guarded (a guarded load sits
                // in a block of its own and waits for all earlier loads, which
                // left one 16-byte load in flight per lane: a token's two
                // passes took ~32 round trips to memory, 8 now).  Batches of 4:
                // with 8 (or 8 in the second pass) the compute waves' bursts
                // slowed the transfer wave's host reads when chunks are small
                // (64-token tiles of 8-token chunks: 2472-2475 against
                // 2431-2442 us), while 4 keeps the example's 32-token chunks
                // at 2470-2475 us (2504-2516 before).
                constexpr int kBatch = 4;
                float ss = 0.f;
#pragma unroll
                for (int j0 = 0; j0 < kRegVecs; j0 += kBatch) {
                    float4 x[kBatch];
#pragma unroll
                    for (int j = 0; j < kBatch; j++) {
                        const uint32_t k = lane + 64u * (uint32_t)(j0 + j);
                        x[j] = t4[k < nv ? k : nv - 1];
                    }
#pragma unroll
                    for (int j = 0; j < kBatch; j++)
                        if (lane + 64u * (uint32_t)(j0 + j) < nv)
                            ss += x[j].x * x[j].x + x[j].y * x[j].y + x[j].z * x[j].z + x[j].w * x[j].w;
                }
                const float r = rsqrtf(wave_sum(ss) / (float)nf + 1e-6f);
                float acc = 0.f;
#pragma unroll
                for (int j0 = 0; j0 < kRegVecs; j0 += kBatch) {
                    float4 x[kBatch];
#pragma unroll
                    for (int j = 0; j < kBatch; j++) {
                        const uint32_t k = lane + 64u * (uint32_t)(j0 + j);
                        x[j] = t4[k < nv ? k : nv - 1];
                    }
#pragma unroll
                    for (int j = 0; j < kBatch; j++) {
                        if (lane + 64u * (uint32_t)(j0 + j) >= nv) continue;
                        const float a = x[j].x * r, b = x[j].y * r, d = x[j].z * r, e = x[j].w * r;
                        acc += sinf(a) * a + sinf(b) * b + sinf(d) * d + sinf(e) * e;
                    }
                }
                acc = wave_sum(acc);
                if (lane == 0) out[c.global_idx((int)i)] = acc;
            }
            return;
        }
        for (uint32_t i = 0; i < c.size; i++) {
            const float* t = c.data<float>((int)i);
            // Whole float4 vectors where the token is 16-byte aligned; the
            // rest (or all of an unaligned token) one float at a time.
            const uint32_t nv = ((uintptr_t)t & 15) == 0 ? nf / 4 : 0;
            const float4* t4 = reinterpret_cast<const float4*>(t);
            float ss = 0.f;
            for (uint32_t k = lane; k < nv; k += 64) {
                const float4 v = t4[k];
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
            for (uint32_t k = nv * 4 + lane; k < nf; k += 64) ss += t[k] * t[k];
            const float r = rsqrtf(wave_sum(ss) / (float)nf + 1e-6f);
            float acc = 0.f;
            for (uint32_t k = lane; k < nv; k += 64) {
                const float4 v = t4[k];
                const float a = v.x * r, b = v.y * r, d = v.z * r, e = v.w * r;
                acc += sinf(a) * a + sinf(b) * b + sinf(d) * d + sinf(e) * e;
            }
            for (uint32_t k = nv * 4 + lane; k < nf; k += 64) {
                const float a = t[k] * r;
                acc += sinf(a) * a;
            }
            acc = wave_sum(acc);
            if (lane == 0) out[c.global_idx((int)i)] = acc;
        }
    }
};
using TokenRmsSin = TokenRmsSinT<false>;

struct NullChunk {
    __device__ void operator()(ChunkView) const {}
};

// list_sums[list_id] += sum of the list's landed bytes read as little-endian
// u32 words (a trailing partial word adds its bytes one by one).  Integer
// sums do not depend on the order of the adds.
struct ListChecksum {
    unsigned long long* list_sums;
    __device__ void operator()(SGListView v) const {
        uint64_t acc = 0;
        for (uint32_t e = 0; e < v.count; e++) {
            const gfd::DeviceSGEntry d = v.get_entry(e);
            const uint8_t* p = reinterpret_cast<const uint8_t*>(d.dst_addr);
            const uint32_t nw = d.size / 4;
            if ((d.dst_addr & 3) == 0) {
                const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
                for (uint32_t k = (uint32_t)v.lane_id; k < nw; k += 64) acc += w[k];
            } else {
                for (uint32_t k = (uint32_t)v.lane_id; k < nw; k += 64)
                    acc += (uint32_t)p[4 * k] | ((uint32_t)p[4 * k + 1] << 8) | ((uint32_t)p[4 * k + 2] << 16) |
                           ((uint32_t)p[4 * k + 3] << 24);
            }
            for (uint32_t b = nw * 4 + (uint32_t)v.lane_id; b < d.size; b += 64) acc += p[b];
        }
        acc = wave_sum(acc);
        if (v.lane_id == 0 && v.list_id < (uint32_t)gfd::MAX_SG_LISTS)
            atomicAdd(&list_sums[v.list_id], (unsigned long long)acc);
    }
};

struct NullList {
    __device__ void operator()(SGListView) const {}
};

// Per entry, the L2 norm of its landed bytes read as fp32, stored at
// out[list_id * count + i] (the MoE consumer of examples/09_sg_warp_spec.cu:
// 44-65).  The wave sums the squares lane-parallel, then across lanes.
// Entries whose destination is not 4-byte aligned, or whose slot lies past
// out_len, are skipped.
struct EntryL2Norm {
    float* out;
    uint32_t out_len;
    __device__ void operator()(SGListView v) const {
        for (uint32_t e = 0; e < v.count; e++) {
            const gfd::DeviceSGEntry d = v.get_entry(e);
            const uint64_t slot = (uint64_t)v.list_id * v.count + e;
            if ((d.dst_addr & 3) != 0 || slot >= out_len) continue;
            const float* x = reinterpret_cast<const float*>(d.dst_addr);
            const uint32_t nf = d.size / 4;
            float acc = 0.f;
            for (uint32_t k = (uint32_t)v.lane_id; k < nf; k += 64) acc = fmaf(x[k], x[k], acc);
            for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
            if (v.lane_id == 0) out[slot] = sqrtf(acc);
        }
    }
};

GFD_WARP_SPEC_KERNEL(ws_token_sum_kernel, TokenSum)
GFD_WARP_SPEC_KERNEL_DB(ws_token_sum_kernel_db, TokenSum)
GFD_WARP_SPEC_KERNEL(ws_rms_sin_kernel, TokenRmsSin)
GFD_WARP_SPEC_KERNEL_DB(ws_rms_sin_kernel_db, TokenRmsSin)
// The same for blocks of at most 9 waves (1 transfer + 2 slots of 4 chunks):
// 3 waves per SIMD leave each ~168 registers, so the consumer holds a whole
// 16 KiB token per wave.
__global__ __launch_bounds__(576) __attribute__((amdgpu_waves_per_eu(1, 3))) void ws_rms_sin_kernel_db9(gfd::TiledQueue* tq, void* gpu_buffer, const void* cpu_base,
                                                             TokenRmsSinT<true> compute_fn) {
    gfd::warp_spec::_warp_spec_tile_loop_double_buffer(tq, gpu_buffer, cpu_base, compute_fn);
}
GFD_WARP_SPEC_KERNEL(ws_null_kernel, NullChunk)
GFD_WARP_SPEC_KERNEL_DB(ws_null_kernel_db, NullChunk)
GFD_SG_WARP_SPEC_KERNEL(sg_checksum_kernel, ListChecksum)
GFD_SG_WARP_SPEC_KERNEL(sg_null_kernel, NullList)
GFD_SG_WARP_SPEC_KERNEL(sg_l2norm_kernel, EntryL2Norm)

// Transfer (wave 0) + compute (wave 1) + submitter (wave 2) + transfer
// helpers (waves 3..) per workgroup, as test/test_sg_gpu_submit.cu:20-213:
// workgroup b submits lists b, b + grid, ... (list i = entries
// [i*epl, (i+1)*epl) of d_entries), waits for all num_lists to land, then
// sets terminate.
template <typename F>
__global__ __launch_bounds__(6 * 64) void sg_gpu_submit_kernel(gfd::DescriptorQueue* dq, gfd::SGTaskQueue* sq, F fn,
                                     const gfd::DeviceSGEntry* d_entries, uint32_t epl, uint32_t num_lists) {
    gfd::sg_warp_spec::_sg_transfer_warp_loop(dq, sq, fn);  // waves 0, 1 and 3.. run here; wave 2 returns
    if (gfd::wave::wave_id() != 2) return;
    gfd::SGDeviceCounters* cnt = gfd::sg_device_counters(sq);
    for (uint32_t l = blockIdx.x; l < num_lists; l += gridDim.x) {
        if (gfd::sg::sg_submit_list(sq, d_entries + (uint64_t)l * epl, epl, l, gfd::SG_FLAG_NONE) == ~0ull) {
            if (gfd::wave::lane_id() == 0)
                __hip_atomic_fetch_or(&cnt->error, gfd::SG_ERR_RING_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
    if (blockIdx.x == 0) {
        if (gfd::sg::sg_wait_gpu_lists_done(sq, num_lists)) {
            gfd::sg::sg_terminate_all_landed(sq);
        } else {
            if (gfd::wave::lane_id() == 0)
                __hip_atomic_fetch_or(&cnt->error, gfd::SG_ERR_LIST_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            gfd::sg::sg_terminate(sq);
        }
    }
}

// Per-launch set-up of an SG session, on the launch stream ahead of the
// session kernel: d_list_done[0 .. MAX_SG_LISTS) zeroed, the device counters
// after them written, trace_words words of trace records zeroed.
__global__ __launch_bounds__(256) void sg_prepare_kernel(uint64_t* d_list_done, gfd::SGDeviceCounters c,
                                                        uint64_t* trace, uint64_t trace_words) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x, n = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t k = i; k < (uint64_t)gfd::MAX_SG_LISTS; k += n) d_list_done[k] = 0;
    if (i == 0) {
        // The launch deadline arrives relative (ticks); it starts now, just
        // ahead of the session kernel on the same stream.
        if (c.deadline) c.deadline += (uint64_t)wall_clock64();
        *reinterpret_cast<gfd::SGDeviceCounters*>(d_list_done + gfd::MAX_SG_LISTS) = c;
    }
    for (uint64_t k = i; k < trace_words; k += n) trace[k] = 0;
}

int fail(int code, const char* what) {
    gfd_internal_set_error(what);
    return code ? code : (int)hipErrorInvalidValue;
}

void fill_ws_result(gfd::WarpSpecSession& s, const gfd::WarpSpecConfig& c, gfd_session_result* r) {
    const auto st = s.get_stats();
    r->units_done = st.descriptors_processed;
    r->bytes = st.bytes_transferred;
    r->lists_done = s.tiles_done();
    r->error_bits = s.error_bits();
    r->elapsed_ms = st.elapsed_ms;
    const auto p = s.get_launch_params();
    r->grid = (int)p.grid;
    r->block = (int)p.block;
    r->tokens_per_chunk = (int)c.effective_tokens_per_chunk();
    r->chunks_per_tile = (int)c.chunks_per_tile();
    r->helper_waves = s.config().helper_waves();
}

gfd::SGWarpSpecSession* S(gfd_sg_session_t s) { return static_cast<gfd::SGWarpSpecSession*>(s); }

}  // namespace

namespace {

// The consumers gfd_warp_spec_run can launch.
enum WsConsumer { kWsNull, kWsTokenSum, kWsRmsSin };

int warp_spec_run(const void* cpu_src, void* gpu_dst, uint32_t total_tokens, uint32_t token_size,
                  uint32_t tokens_per_tile, uint32_t tokens_per_chunk, int double_buffer, int per_tile_mode,
                  int num_blocks, int helper_waves, WsConsumer consumer, float* out, int iters, double* kernel_ms,
                  gfd_session_result* res) {
    if (!cpu_src || !gpu_dst || total_tokens == 0 || token_size == 0 || iters < 1 || !res ||
        (consumer != kWsNull && !out))
        return fail(hipErrorInvalidValue, "gfd_warp_spec_run: invalid argument");
    gfd::WarpSpecConfig c;
    c.total_tokens = total_tokens;
    c.token_size = token_size;
    c.cpu_src = const_cast<void*>(cpu_src);
    c.gpu_dst = gpu_dst;
    c.tokens_per_tile = tokens_per_tile;
    c.tokens_per_chunk = tokens_per_chunk;
    c.double_buffer = double_buffer != 0;
    c.per_tile_mode = per_tile_mode != 0;
    c.num_blocks = num_blocks;
    if (helper_waves >= 0) c.transfer_helper_waves = helper_waves;
    if (c.tokens_per_tile == 0 || c.effective_tokens_per_chunk() == 0 ||
        c.tokens_per_tile % c.effective_tokens_per_chunk() != 0 || c.block_size() > 1024 ||
        c.chunks_per_tile() > (uint32_t)gfd::warp_spec::MAX_CHUNKS_PER_TILE)
        return fail(hipErrorInvalidValue, "gfd_warp_spec_run: tile / chunk shape not supported");
    gfd::WarpSpecSession s(c);
    if (!s.ok()) return fail(hipErrorInvalidValue, "gfd_warp_spec_run: session construction failed");
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        return fail(hipErrorOutOfMemory, "gfd_warp_spec_run: event creation failed");
    int rc = 0;
    const auto p = s.get_launch_params();
    for (int it = 0; it < iters && rc == 0; it++) {
        // launch() with the HIP events around the kernel alone: before_launch
        // clears the signals with a blocking memset first.
        s.before_launch(nullptr);
        (void)hipEventRecord(e0, nullptr);
        if (consumer == kWsTokenSum) {
            if (c.double_buffer)
                hipLaunchKernelGGL(ws_token_sum_kernel_db, dim3(p.grid), dim3(p.block), 0, nullptr, p.tq, p.gpu_buffer,
                                   p.cpu_base, TokenSum{out});
            else
                hipLaunchKernelGGL(ws_token_sum_kernel, dim3(p.grid), dim3(p.block), 0, nullptr, p.tq, p.gpu_buffer,
                                   p.cpu_base, TokenSum{out});
        } else if (consumer == kWsRmsSin) {
            if (c.double_buffer && p.block <= 576)
                hipLaunchKernelGGL(ws_rms_sin_kernel_db9, dim3(p.grid), dim3(p.block), 0, nullptr, p.tq, p.gpu_buffer,
                                   p.cpu_base, TokenRmsSinT<true>{out});
            else if (c.double_buffer)
                hipLaunchKernelGGL(ws_rms_sin_kernel_db, dim3(p.grid), dim3(p.block), 0, nullptr, p.tq, p.gpu_buffer,
                                   p.cpu_base, TokenRmsSin{out});
            else
                hipLaunchKernelGGL(ws_rms_sin_kernel, dim3(p.grid), dim3(p.block), 0, nullptr, p.tq, p.gpu_buffer,
                                   p.cpu_base, TokenRmsSin{out});
        } else {
            if (c.double_buffer)
                hipLaunchKernelGGL(ws_null_kernel_db, dim3(p.grid), dim3(p.block), 0, nullptr, p.tq, p.gpu_buffer,
                                   p.cpu_base, NullChunk{});
            else
                hipLaunchKernelGGL(ws_null_kernel, dim3(p.grid), dim3(p.block), 0, nullptr, p.tq, p.gpu_buffer,
                                   p.cpu_base, NullChunk{});
        }
        (void)hipEventRecord(e1, nullptr);
        const hipError_t le = hipGetLastError();
        const bool ok = s.synchronize();
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (kernel_ms) kernel_ms[it] = ms;
        if (le != hipSuccess) rc = fail(le, "gfd_warp_spec_run: launch failed");
        else if (!ok) rc = fail(hipErrorLaunchFailure, "gfd_warp_spec_run: kernel reported an error or missing tiles");
    }
    fill_ws_result(s, c, res);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

}  // namespace

extern "C" int gfd_warp_spec_run(const void* cpu_src, void* gpu_dst, uint32_t total_tokens, uint32_t token_size,
                                 uint32_t tokens_per_tile, uint32_t tokens_per_chunk, int double_buffer,
                                 int per_tile_mode, int num_blocks, int helper_waves, float* token_sums, int iters,
                                 double* kernel_ms, gfd_session_result* res) {
    return warp_spec_run(cpu_src, gpu_dst, total_tokens, token_size, tokens_per_tile, tokens_per_chunk, double_buffer,
                         per_tile_mode, num_blocks, helper_waves, token_sums ? kWsTokenSum : kWsNull, token_sums,
                         iters, kernel_ms, res);
}

extern "C" int gfd_warp_spec_run_rms_sin(const void* cpu_src, void* gpu_dst, uint32_t total_tokens,
                                         uint32_t token_size, uint32_t tokens_per_tile, uint32_t tokens_per_chunk,
                                         int double_buffer, int num_blocks, int helper_waves, float* out, int iters,
                                         double* kernel_ms, gfd_session_result* res) {
    if (token_size % 4 != 0)
        return fail(hipErrorInvalidValue, "gfd_warp_spec_run_rms_sin: tokens must be whole floats");
    return warp_spec_run(cpu_src, gpu_dst, total_tokens, token_size, tokens_per_tile, tokens_per_chunk, double_buffer,
                         0, num_blocks, helper_waves, kWsRmsSin, out, iters, kernel_ms, res);
}

extern "C" int gfd_sg_session_create(int num_compute_warps, int num_blocks, uint32_t idle_limit_ms, int helper_waves,
                                     gfd_sg_session_t* out) {
    if (!out) return fail(hipErrorInvalidValue, "gfd_sg_session_create: out is NULL");
    gfd::SGWarpSpecConfig c;
    c.num_compute_warps = num_compute_warps;
    c.num_blocks = num_blocks;
    c.idle_limit_ms = idle_limit_ms;
    if (helper_waves >= 0) c.transfer_helper_waves = helper_waves;
    auto* s = new gfd::SGWarpSpecSession(c);
    if (!s->ok()) {
        delete s;
        return fail(hipErrorInvalidValue, "gfd_sg_session_create: session construction failed");
    }
    *out = s;
    return 0;
}

extern "C" void gfd_sg_session_destroy(gfd_sg_session_t s) { delete S(s); }

extern "C" int64_t gfd_sg_session_submit(gfd_sg_session_t s, const gfd_device_sg_entry* entries, uint32_t count,
                                         uint32_t list_id, uint32_t flags) {
    if (!s) return -1;
    const uint64_t idx =
        S(s)->submit_sg_list(reinterpret_cast<const gfd::DeviceSGEntry*>(entries), count, list_id, flags);
    if (idx == ~0ull) {
        fail(hipErrorInvalidValue, "gfd_sg_session_submit: rejected (invalid argument, or ring / pool full)");
        return -1;
    }
    return (int64_t)idx;
}

extern "C" int gfd_sg_session_launch(gfd_sg_session_t s, unsigned long long* list_sums, void* stream) {
    if (!s) return fail(hipErrorInvalidValue, "gfd_sg_session_launch: NULL session");
    if (list_sums) S(s)->launch(sg_checksum_kernel, ListChecksum{list_sums}, stream);
    else S(s)->launch(sg_null_kernel, NullList{}, stream);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(e, "gfd_sg_session_launch: launch failed");
}

extern "C" int gfd_sg_session_launch_l2norm(gfd_sg_session_t s, float* out, uint32_t out_len, void* stream) {
    if (!s || !out) return fail(hipErrorInvalidValue, "gfd_sg_session_launch_l2norm: NULL argument");
    S(s)->launch(sg_l2norm_kernel, EntryL2Norm{out, out_len}, stream);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(e, "gfd_sg_session_launch_l2norm: launch failed");
}

extern "C" int gfd_sg_session_launch_gpu_submit(gfd_sg_session_t s, const gfd_device_sg_entry* d_entries,
                                                uint32_t entries_per_list, uint32_t num_lists,
                                                unsigned long long* list_sums, void* stream) {
    if (!s || !d_entries || entries_per_list == 0 || num_lists == 0 ||
        entries_per_list > (uint32_t)gfd::MAX_SG_POOL_ENTRIES || num_lists > (uint32_t)gfd::MAX_SG_LISTS)
        return fail(hipErrorInvalidValue, "gfd_sg_session_launch_gpu_submit: invalid argument");
    gfd::SGWarpSpecSession* p = S(s);
    const int helpers = p->helper_waves();
    // Every list comes from the kernel's own submitters: a stall anywhere
    // ends the launch at the deadline with error bits.
    p->before_launch(stream, helpers, -1, p->idle_limit_ms());
    const auto* ents = reinterpret_cast<const gfd::DeviceSGEntry*>(d_entries);
    const dim3 grid((unsigned)p->num_blocks()), block((unsigned)(3 + helpers) * 64);
    if (list_sums)
        hipLaunchKernelGGL(sg_gpu_submit_kernel<ListChecksum>, grid, block, 0, (hipStream_t)stream, p->get_desc_queue(),
                           p->get_sg_queue(), ListChecksum{list_sums}, ents, entries_per_list, num_lists);
    else
        hipLaunchKernelGGL(sg_gpu_submit_kernel<NullList>, grid, block, 0, (hipStream_t)stream, p->get_desc_queue(),
                           p->get_sg_queue(), NullList{}, ents, entries_per_list, num_lists);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(e, "gfd_sg_session_launch_gpu_submit: launch failed");
}

extern "C" int gfd_sg_prepare_launch(uint64_t* d_list_done, const void* counters, uint64_t* trace,
                                     uint64_t trace_words, gfd_stream_t stream) {
    if (!d_list_done || !counters || (trace_words && !trace)) return (int)hipErrorInvalidValue;
    gfd::SGDeviceCounters c;
    std::memcpy(&c, counters, sizeof(c));
    hipLaunchKernelGGL(sg_prepare_kernel, dim3(4), dim3(256), 0, (hipStream_t)stream, d_list_done, c, trace,
                       trace_words);
    return (int)hipGetLastError();
}

extern "C" int gfd_sg_session_synchronize(gfd_sg_session_t s, uint64_t extra_gpu_lists) {
    if (!s) return fail(hipErrorInvalidValue, "gfd_sg_session_synchronize: NULL session");
    return S(s)->synchronize(extra_gpu_lists) ? 0 : fail(hipErrorLaunchFailure, "gfd_sg_session_synchronize: lists did not land or the kernel reported an error");
}

extern "C" int gfd_sg_session_reset(gfd_sg_session_t s) {
    if (!s) return fail(hipErrorInvalidValue, "gfd_sg_session_reset: NULL session");
    S(s)->reset();
    return 0;
}

extern "C" int gfd_sg_session_stats(gfd_sg_session_t s, gfd_session_result* r) {
    if (!s || !r) return fail(hipErrorInvalidValue, "gfd_sg_session_stats: invalid argument");
    const auto st = S(s)->get_stats();
    *r = gfd_session_result{};
    r->units_done = st.descriptors_processed;
    r->bytes = st.bytes_transferred;
    r->lists_done = S(s)->lists_landed();
    r->error_bits = S(s)->error_bits();
    r->elapsed_ms = st.elapsed_ms;
    r->grid = S(s)->num_blocks();
    r->block = S(s)->block_size();
    r->helper_waves = S(s)->helper_waves();
    return 0;
}

extern "C" void* gfd_sg_session_queue(gfd_sg_session_t s) { return s ? (void*)S(s)->get_sg_queue() : nullptr; }

static_assert(sizeof(gfd_sg_trace_list) == sizeof(gfd::SGTraceList), "gfd_sg_trace_list must match gfd::SGTraceList");
static_assert(sizeof(gfd_sg_trace_block) == sizeof(gfd::SGTraceBlock), "gfd_sg_trace_block must match gfd::SGTraceBlock");

extern "C" int gfd_sg_session_enable_trace(gfd_sg_session_t s, uint32_t max_lists) {
    if (!s) return fail(hipErrorInvalidValue, "gfd_sg_session_enable_trace: NULL session");
    return S(s)->enable_trace(max_lists) ? 0 : fail(hipErrorOutOfMemory, "gfd_sg_session_enable_trace: allocation failed");
}

extern "C" int gfd_sg_session_read_trace(gfd_sg_session_t s, gfd_sg_trace_list* lists, uint32_t max_lists,
                                         gfd_sg_trace_block* blocks, uint32_t max_blocks, uint32_t* n_lists,
                                         uint32_t* n_blocks) {
    if (!s || !n_lists || !n_blocks || (max_lists && !lists) || (max_blocks && !blocks))
        return fail(hipErrorInvalidValue, "gfd_sg_session_read_trace: invalid argument");
    std::vector<gfd::SGTraceList> l;
    std::vector<gfd::SGTraceBlock> b;
    if (!S(s)->read_trace(l, b))
        return fail(hipErrorNotReady, "gfd_sg_session_read_trace: tracing is off, the launch is still running, or the copy failed");
    *n_lists = (uint32_t)std::min<size_t>(l.size(), max_lists);
    *n_blocks = (uint32_t)std::min<size_t>(b.size(), max_blocks);
    if (*n_lists) std::memcpy(lists, l.data(), *n_lists * sizeof(gfd_sg_trace_list));
    if (*n_blocks) std::memcpy(blocks, b.data(), *n_blocks * sizeof(gfd_sg_trace_block));
    return 0;
}

// Host-submitted SG transfer timed from launch until the host has seen every
// list land (done markers), then terminate + sync.  times_us[iters].
extern "C" int gfd_bench_sg_session(gfd_sg_session_t s, const gfd_device_sg_entry* entries, uint32_t count,
                                    uint32_t entries_per_list, int warmup, int iters, double* times_us) {
    if (!s || !entries || count == 0 || entries_per_list == 0 || iters < 1 || !times_us ||
        count > (uint32_t)gfd::MAX_SG_POOL_ENTRIES ||
        (count + entries_per_list - 1) / entries_per_list > (uint32_t)gfd::MAX_SG_LISTS)
        return fail(hipErrorInvalidValue,
                    "gfd_bench_sg_session: invalid argument (at most 16384 entries in at most 512 lists)");
    gfd::SGWarpSpecSession* p = S(s);
    const uint32_t nl = (count + entries_per_list - 1) / entries_per_list;
    for (int it = -warmup; it < iters; it++) {
        p->reset();
        for (uint32_t l = 0; l < nl; l++) {
            const uint32_t b = l * entries_per_list, n = std::min(entries_per_list, count - b);
            if (p->submit_sg_list(reinterpret_cast<const gfd::DeviceSGEntry*>(entries) + b, n, l) == ~0ull)
                return fail(hipErrorInvalidValue, "gfd_bench_sg_session: submit rejected");
        }
        gfd::SGTaskQueue* sq = p->get_sg_queue();
        const auto t0 = std::chrono::steady_clock::now();
        p->launch(sg_null_kernel, NullList{}, nullptr);
        // Spin until every list's done marker is up (bounded: 10 s).
        bool all = false;
        while (!all) {
            all = true;
            for (uint64_t i = 0; i < nl; i++)
                if (__atomic_load_n(const_cast<uint64_t*>(&sq->lists[i].done), __ATOMIC_ACQUIRE) < i + 1) {
                    all = false;
                    break;
                }
            if (std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > 10.0) break;
        }
        const auto t1 = std::chrono::steady_clock::now();
        if (!p->synchronize() || !all) return fail(hipErrorLaunchFailure, "gfd_bench_sg_session: lists did not land");
        if (it >= 0) times_us[it] = std::chrono::duration<double, std::micro>(t1 - t0).count();
    }
    return 0;
}
