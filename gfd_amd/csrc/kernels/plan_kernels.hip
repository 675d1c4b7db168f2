// GPU-built SG lists for GFD Direct: the pattern of the reference's
// examples/03_gpu_planned_transfer.cu:32-66, where kernels select the tokens
// routed to one expert and write the SGEntry list straight into pinned host
// memory, and the host then hands that list to submit_direct.
//
// MI355X design: one workgroup of 16 waves walks the routing table in tiles
// of 1024 tokens.  Each wave ballots its matches, and the per-wave counts
// (in LDS) give every match its slot, so the list is in token order (stable)
// and the same on every run.  The reference compacts with an atomicAdd per
// match, which orders slots by arrival.  One workgroup moves ~1 us per tile:
// enough for routing tables of a few thousand tokens, the planner's use.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gfd_capi.h"

namespace {

constexpr int kPlanBlock = 1024;

__global__ __launch_bounds__(kPlanBlock) void plan_expert_entries_kernel(
    const int* __restrict__ routing, int num_tokens, int expert, uint64_t cpu_base, uint64_t stride,
    uint64_t gpu_dst, uint64_t token_size, gfd_sg_entry* __restrict__ entries, int* __restrict__ count) {
    __shared__ int wave_total[kPlanBlock / 64];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = (int)(blockDim.x >> 6);
    int base = 0;
    for (int t0 = 0; t0 < num_tokens; t0 += (int)blockDim.x) {
        const int t = t0 + tid;
        const bool hit = t < num_tokens && routing[t] == expert;
        const uint64_t mask = __ballot(hit);
        const int before = __popcll(mask & ((1ull << lane) - 1ull));
        if (lane == 0) wave_total[wave] = __popcll(mask);
        __syncthreads();
        int off = 0, tile = 0;
        for (int w = 0; w < nwaves; w++) {
            const int c = wave_total[w];
            off += w < wave ? c : 0;
            tile += c;
        }
        if (hit) {
            const uint64_t k = (uint64_t)(base + off + before);
            gfd_sg_entry e;
            e.dst = gpu_dst + k * token_size;
            e.src = cpu_base + (uint64_t)t * stride;
            e.size = token_size;
            entries[k] = e;
        }
        base += tile;
        __syncthreads();  // wave_total is rewritten by the next tile
    }
    if (tid == 0) *count = base;
}

}  // namespace

extern "C" int gfd_plan_expert_entries(const int* routing, int num_tokens, int expert, const void* cpu_base,
                                       uint64_t stride, void* gpu_dst, uint32_t token_size, gfd_sg_entry* entries,
                                       int* count, void* stream) {
    if (!routing || !entries || !count || num_tokens < 0 || token_size == 0)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(plan_expert_entries_kernel, dim3(1), dim3(kPlanBlock), 0, (hipStream_t)stream, routing,
                       num_tokens, expert, (uint64_t)(uintptr_t)cpu_base, stride, (uint64_t)(uintptr_t)gpu_dst,
                       (uint64_t)token_size, entries, count);
    return (int)hipGetLastError();
}
