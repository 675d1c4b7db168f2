// MoE-routed scattered gather with a wave-specialised RMSNorm consumer (gfx950).
//
// Role in the reference: the SG warp-specialised path (include/gfd/sg_warp_spec.cuh:
// a transfer warp turns per-expert (src, dst, size) lists into copies, a compute
// warp runs a functor on each list once it has landed; examples/09_sg_warp_spec.cu
// builds the lists on the GPU).  Here the whole path stays on the GPU:
//
//   1. moe_top2_kernel   — top-2 experts per token from the logits (ties go to
//                          the lower expert id), one wave64 per token.
//   2. moe_lists_kernel  — one workgroup per expert builds its row list in token
//                          order (stable; no atomics), plus the expert offsets.
//                          Rows are packed expert-major.
//   3. sg_gather_norm_kernel<P, C, V> — per workgroup, P producer waves read whole
//                          rows straight from pinned host memory (16-byte loads
//                          over PCIe), write them to HBM and into an LDS ring of
//                          S row slots; C consumer waves wait on the slot flags
//                          (LDS acquire + s_sleep), compute a bf16 RMSNorm of the
//                          row in fp32 and write it to HBM, then free the slot.
//                          C = 0 is the pure-transfer variant.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "capi_error.h"
#include "gfd/wave_ops.h"
#include "gfd_capi.h"

// Scratch of gfd_moe_route_noalloc: the top-2 expert pairs between its two
// kernels, for up to kNoAllocMaxTokens tokens (512 KiB per GPU, held until the
// process ends).  Host code never uses this name as an address: each
// device's copy is reached through the pointer hipGetSymbolAddress returns
// for it (moe_scratch_ptr below).
constexpr int kNoAllocMaxTokens = 65536;
static __device__ __align__(256) int scratch[2 * kNoAllocMaxTokens];

namespace {

constexpr int kWave = 64;
constexpr int kSlots = 4;              // LDS ring depth per workgroup
constexpr int kMaxRowBytes = 14336;    // 7168 bf16
constexpr uint64_t kSpinLimit = 1ull << 26;  // LDS flag polls before giving up

// ---------------------------------------------------------------- routing

__device__ __forceinline__ void wave_argmax(float& v, int& idx) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, kWave);
        const int oi = __shfl_xor(idx, off, kWave);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
}

__global__ __launch_bounds__(256) void moe_top2_kernel(const float* __restrict__ logits, int num_tokens,
                                                       int num_experts, int* __restrict__ top2) {
    const int t = (int)((blockIdx.x * blockDim.x + threadIdx.x) / kWave);
    const int lane = (int)(threadIdx.x % kWave);
    if (t >= num_tokens) return;  // uniform per wave
    const float x = lane < num_experts ? logits[(size_t)t * num_experts + lane] : -INFINITY;
    float v = x;
    int i = lane;
    wave_argmax(v, i);
    const int first = i;
    v = (lane == first || lane >= num_experts) ? -INFINITY : x;
    i = lane;
    wave_argmax(v, i);
    if (lane == 0) {
        top2[2 * t] = first;
        top2[2 * t + 1] = i;
    }
}

// Workgroup e: offsets[e] = number of (token, choice) pairs routed to experts
// below e; row_token[offsets[e] + k] = k-th token (in token order) routed to e.
__global__ __launch_bounds__(256) void moe_lists_kernel(const int* __restrict__ top2, int num_tokens,
                                                        int num_experts, int* __restrict__ offsets,
                                                        int* __restrict__ row_token) {
    __shared__ int wave_sum[4];
    __shared__ int block_base;
    const int e = (int)blockIdx.x;
    const int tid = (int)threadIdx.x;
    const int lane = tid % kWave, wave = tid / kWave;

    // Offset of this expert: pairs routed to lower experts.
    int below = 0;
    for (int t = tid; t < num_tokens; t += 256) below += (top2[2 * t] < e) + (top2[2 * t + 1] < e);
    for (int off = 32; off >= 1; off >>= 1) below += __shfl_xor(below, off, kWave);
    if (lane == 0) wave_sum[wave] = below;
    __syncthreads();
    if (tid == 0) {
        block_base = wave_sum[0] + wave_sum[1] + wave_sum[2] + wave_sum[3];
        offsets[e] = block_base;
        if (e == num_experts - 1) offsets[num_experts] = 2 * num_tokens;
    }
    __syncthreads();

    // Stable placement: block-wide exclusive prefix over token order.
    int running = block_base;
    for (int base = 0; base < num_tokens; base += 256) {
        const int t = base + tid;
        const bool hit = t < num_tokens && (top2[2 * t] == e || top2[2 * t + 1] == e);
        const uint64_t mask = __ballot(hit);
        const int before_in_wave = __popcll(mask & ((1ull << lane) - 1ull));
        __syncthreads();
        if (lane == 0) wave_sum[wave] = __popcll(mask);
        __syncthreads();
        int before_waves = 0;
        for (int w = 0; w < wave; w++) before_waves += wave_sum[w];
        if (hit) row_token[running + before_waves + before_in_wave] = t;
        running += wave_sum[0] + wave_sum[1] + wave_sum[2] + wave_sum[3];
    }
}

// ------------------------------------------------------ gather + RMSNorm

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Round-to-nearest-even fp32 -> bf16 (finite values).
__device__ __forceinline__ uint32_t to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ int lds_load_acquire(int* p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void lds_store_release(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Wait until *flag == want; false if the spin limit ran out (the caller then
// skips its row and reports the error instead of hanging the workgroup).
__device__ __forceinline__ bool lds_wait(int* flag, int want) {
    for (uint64_t n = 0; n < kSpinLimit; n++) {
        if (lds_load_acquire(flag) == want) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

// Workgroup b owns rows [b*R/G, (b+1)*R/G) of the expert-major row order.
// Row r copies token row_token[r] (host_base + token * token_stride,
// row_bytes = V * 1 KiB) to dst + r * row_bytes; with C > 0 it also writes
// RMSNorm(row) (bf16, weight w, epsilon eps) to out + r * row_bytes.
//
// V (16-byte vectors per lane) is a template parameter so that every lane's
// V loads are straight-line code: a guarded load sits in its own basic block,
// and the compiler then waits for all earlier loads before issuing it.  The
// vectors are native clang vectors so that they stay in registers.
template <int P, int C, int V>
__global__ __launch_bounds__(kWave*(P + C)) void sg_gather_norm_kernel(
    const uint8_t* __restrict__ host_base, uint64_t token_stride, int num_tokens, const int* __restrict__ row_token,
    int num_rows, uint8_t* __restrict__ dst, uint8_t* __restrict__ out, const uint16_t* __restrict__ weight,
    float eps, int* __restrict__ error_flag) {
    using gfd::wave::vec4u;
    constexpr uint32_t row_bytes = (uint32_t)V * kWave * 16;
    __shared__ vec4u ring[C > 0 ? kSlots : 1][V * kWave];
    __shared__ vec4u wlds[C > 0 ? V * kWave : 1];  // RMSNorm weights, staged once per workgroup
    __shared__ int slot_row[kSlots];
    const int wave = (int)(threadIdx.x / kWave);
    const int lane = (int)(threadIdx.x % kWave);
    const int r0 = (int)(((int64_t)blockIdx.x * num_rows) / gridDim.x);
    const int r1 = (int)(((int64_t)(blockIdx.x + 1) * num_rows) / gridDim.x);
    const int rows = r1 - r0;

    if (C > 0) {
        if (threadIdx.x < kSlots) slot_row[threadIdx.x] = 0;
        for (uint32_t k = threadIdx.x; k < (uint32_t)(V * kWave); k += blockDim.x)
            wlds[k] = gfd::wave::gload((uint64_t)(uintptr_t)weight + (uint64_t)k * 16);
        __syncthreads();
    }

    if (wave < P) {
        // ---------------- producer waves
        for (int i = wave; i < rows; i += P) {
            const int r = r0 + i;
            const int s = i % kSlots;
            if (C > 0 && !lds_wait(&slot_row[s], 0)) {
                if (lane == 0) atomicOr(error_flag, 1);
                return;
            }
            const int tok = row_token[r];
            if (tok < 0 || tok >= num_tokens) {  // not a valid token: report, keep the ring moving
                if (lane == 0) atomicOr(error_flag, 4);
                if (C > 0) lds_store_release(&slot_row[s], i + 1);
                continue;
            }
            const uint64_t src = (uint64_t)(uintptr_t)host_base + (uint64_t)tok * token_stride;
            const uint64_t d = (uint64_t)(uintptr_t)dst + (uint64_t)r * row_bytes;
            vec4u v[V];
#pragma unroll
            for (int k = 0; k < V; k++) v[k] = gfd::wave::gload(src + (uint64_t)(k * kWave + lane) * 16);
#pragma unroll
            for (int k = 0; k < V; k++) gfd::wave::gstore(d + (uint64_t)(k * kWave + lane) * 16, v[k]);
            if (C > 0) {
#pragma unroll
                for (int k = 0; k < V; k++) ring[s][k * kWave + lane] = v[k];
                lds_store_release(&slot_row[s], i + 1);
            }
        }
    } else if (C > 0) {
        // ---------------- consumer waves
        const int c = wave - P;
        const float inv_dim = 1.0f / (float)(row_bytes / 2);
        for (int i = c; i < rows; i += C) {
            const int r = r0 + i;
            const int s = i % kSlots;
            if (!lds_wait(&slot_row[s], i + 1)) {
                if (lane == 0) atomicOr(error_flag, 2);
                return;
            }
            vec4u x[V];
            float ss = 0.f;
#pragma unroll
            for (int k = 0; k < V; k++) {
                x[k] = ring[s][k * kWave + lane];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float a = bf16_lo(x[k][j]), b = bf16_hi(x[k][j]);
                    ss += a * a + b * b;
                }
            }
            lds_store_release(&slot_row[s], 0);  // row is in registers: free the slot
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, kWave);
            const float scale = 1.0f / sqrtf(ss * inv_dim + eps);
            const uint64_t o = (uint64_t)(uintptr_t)out + (uint64_t)r * row_bytes;
#pragma unroll
            for (int k = 0; k < V; k++) {
                const vec4u wk = wlds[k * kWave + lane];
                vec4u y;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float lo = bf16_lo(x[k][j]) * scale * bf16_lo(wk[j]);
                    const float hi = bf16_hi(x[k][j]) * scale * bf16_hi(wk[j]);
                    y[j] = to_bf16(lo) | (to_bf16(hi) << 16);
                }
                gfd::wave::gstore(o + (uint64_t)(k * kWave + lane) * 16, y);
            }
        }
    }
}

template <int V>
void launch_gather_norm(const void* host_base, uint64_t token_stride, int num_tokens, const int* row_token,
                        int num_rows, void* dst, void* out, const uint16_t* weight, float eps, int num_blocks,
                        int* error_flag, hipStream_t st) {
    if (out)
        hipLaunchKernelGGL((sg_gather_norm_kernel<4, 4, V>), dim3(num_blocks), dim3(kWave * 8), 0, st,
                           (const uint8_t*)host_base, token_stride, num_tokens, row_token, num_rows, (uint8_t*)dst,
                           (uint8_t*)out, weight, eps, error_flag);
    else
        hipLaunchKernelGGL((sg_gather_norm_kernel<4, 0, V>), dim3(num_blocks), dim3(kWave * 4), 0, st,
                           (const uint8_t*)host_base, token_stride, num_tokens, row_token, num_rows, (uint8_t*)dst,
                           (uint8_t*)nullptr, weight, eps, error_flag);
}

int g_cus = 0;
int cus() {
    if (!g_cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || g_cus <= 0)
            g_cus = 256;
    }
    return g_cus;
}

// Device address of this device's `scratch`, looked up once per device with
// that device current; 0 or a HIP error.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int moe_scratch_ptr(int** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<int*>(g_scratch_ptr[dev]);
    return 0;
}

int launch_route(const float* logits, int num_tokens, int num_experts, int* top2, int* offsets, int* row_token,
                 hipStream_t st) {
    const int waves_per_block = 256 / kWave;
    hipLaunchKernelGGL(moe_top2_kernel, dim3((num_tokens + waves_per_block - 1) / waves_per_block), dim3(256), 0, st,
                       logits, num_tokens, num_experts, top2);
    hipLaunchKernelGGL(moe_lists_kernel, dim3(num_experts), dim3(256), 0, st, top2, num_tokens, num_experts, offsets,
                       row_token);
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int gfd_moe_route_noalloc(const float* logits, int num_tokens, int num_experts, int* offsets,
                                     int* row_token, void* stream) {
    if (num_tokens <= 0 || num_experts < 2 || num_experts > 64 || !logits || !offsets || !row_token) {
        gfd_internal_set_error("gfd_moe_route_noalloc: invalid argument");
        return (int)hipErrorInvalidValue;
    }
    if (num_tokens > kNoAllocMaxTokens) {
        gfd_internal_set_error("gfd_moe_route_noalloc: num_tokens exceeds the scratch maximum of 65536 tokens");
        return (int)hipErrorInvalidValue;
    }
    int* top2 = nullptr;
    const int rc = moe_scratch_ptr(&top2);
    if (rc != 0) {
        gfd_internal_set_error("gfd_moe_route_noalloc: hipGetSymbolAddress of the scratch array failed");
        return rc;
    }
    return launch_route(logits, num_tokens, num_experts, top2, offsets, row_token, (hipStream_t)stream);
}

extern "C" int gfd_moe_route(const float* logits, int num_tokens, int num_experts, int* top2, int* offsets,
                             int* row_token, void* stream) {
    if (num_tokens <= 0 || num_experts < 2 || num_experts > 64 || !logits || !top2 || !offsets || !row_token)
        return (int)hipErrorInvalidValue;
    return launch_route(logits, num_tokens, num_experts, top2, offsets, row_token, (hipStream_t)stream);
}

extern "C" int gfd_sg_gather_rmsnorm(const void* host_base, uint64_t token_stride, int num_tokens, const int* row_token,
                                     int num_rows, uint32_t row_bytes, void* dst, void* out, const uint16_t* weight,
                                     float eps, int num_blocks, int* error_flag, void* stream) {
    if (num_rows < 0 || num_tokens <= 0 || !host_base || !row_token || !dst || !error_flag || row_bytes == 0 ||
        row_bytes % (kWave * 16) != 0 || row_bytes > (uint32_t)kMaxRowBytes || (out && !weight))
        return (int)hipErrorInvalidValue;
    if (num_rows == 0) return 0;
    // Default: 64 workgroups (256 producer waves, 14 loads in flight per lane,
    // ~3.5 MiB of host reads outstanding).  Measured on MI355X for 8192 rows
    // of 14 KiB: 57.7 GB/s at 32-96 workgroups, 55 GB/s at 192-256.
    if (num_blocks <= 0) num_blocks = cus() < 64 ? cus() : 64;
    if (num_blocks > num_rows) num_blocks = num_rows;
    hipStream_t st = (hipStream_t)stream;
    switch (row_bytes / (kWave * 16)) {
#define GFD_ROW_CASE(v)                                                                                          \
    case v:                                                                                                      \
        launch_gather_norm<v>(host_base, token_stride, num_tokens, row_token, num_rows, dst, out, weight, eps, \
                              num_blocks, error_flag, st);                                                      \
        break;
        GFD_ROW_CASE(1) GFD_ROW_CASE(2) GFD_ROW_CASE(3) GFD_ROW_CASE(4) GFD_ROW_CASE(5) GFD_ROW_CASE(6)
        GFD_ROW_CASE(7) GFD_ROW_CASE(8) GFD_ROW_CASE(9) GFD_ROW_CASE(10) GFD_ROW_CASE(11) GFD_ROW_CASE(12)
        GFD_ROW_CASE(13) GFD_ROW_CASE(14)
#undef GFD_ROW_CASE
        default:
            return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}
