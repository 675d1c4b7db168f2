// The MoE-routed gather (top-2 of 64 experts, 14 KiB bf16 rows) through
// SGWarpSpecSession, as the reference runs its SG MoE example: per-expert
// (src, dst, size) lists are built on the GPU by submitter waves and posted
// with the sg:: primitives (the pattern of examples/09_sg_warp_spec.cu:78-294
// and test/test_sg_gpu_submit.cu:20-213), the session's transfer waves copy
// each list from pinned host memory to HBM (include/gfd/sg_warp_spec.h), and
// the compute waves run the consumer: a per-row bf16 RMSNorm, or nothing
// (pure transfer).  The RMSNorm takes each row from the LDS ring the transfer
// wave stages it in (the session's staged-row mode) as soon as the row is
// copied; with GFD_SG_STAGED_ROWS=0 it runs per landed list instead, reading
// the rows back from HBM.
//
// Lists: expert e's rows [offsets[e], offsets[e+1]) in the expert-major order
// of gfd_moe_route, cut into lists of at most rows_per_list (<= 64) rows, so
// a workgroup gets several lists and the RMSNorm of one overlaps the copy of
// the next.  List ids run 0 .. total-1: first every expert's full lists, in
// expert order, then every expert's shorter remainder list, longest first
// (ties in expert order) (lists past
// MAX_SG_LISTS reuse ring slots once landed; ids from MAX_SG_LISTS on have no
// d_list_done word, which the kernel does not need).  Entry k of the
// list for rows [r, r + n): src = host_base + row_token[r + k] * token_stride,
// dst = dst + (r + k) * row_bytes, size = row_bytes, tag = r + k (the row).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "bf16_ops.h"
#include "capi_error.h"
#include "gfd/sg_device_primitives.h"
#include "gfd/sg_warp_spec.h"
#include "gfd/warp_spec_session.h"
#include "gfd_capi.h"

namespace {

using gfd::sg_warp_spec::SGListView;

// y = x / sqrt(mean(x^2) + eps) * w per landed row, fp32 arithmetic, bf16
// round-to-nearest-even out, to out + row * row_bytes (the entry's tag is the
// row).  V = row_bytes / 1 KiB vectors per lane.
//
// Staged rows: the row is read from the LDS slot, the slot handed back, and
// the weights (loaded on the wave's first row and parked in LDS, each lane
// reading back only the vectors it stored itself: in registers they would
// not fit beside a row and its fp32 values) applied on the way out.
//
// List mode: the rows were just written to HBM by the transfer waves of this
// workgroup, so a row's own arithmetic is short and its latency is what
// counts.  Per list: up to 64 entries are read in one request (lane i reads
// entry i) instead of one round trip per row, and the weights are loaded
// once per list into the same LDS copy.
//
// In both, entries whose size is not row_bytes (rows skipped for a bad token
// id have size 0) are left alone.
template <int V>
__device__ __forceinline__ float sum_squares(const gfd::wave::vec4u (&x)[V]) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < V; k++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float a = gfd::bf16::lo(x[k][j]), b = gfd::bf16::hi(x[k][j]);
            ss += a * a + b * b;
        }
    return ss;
}

template <int V>
__device__ __forceinline__ void store_normalised(const gfd::wave::vec4u (&x)[V], const gfd::wave::vec4u* w_lds,
                                                 float scale, uint64_t o, uint32_t lane) {
    using gfd::wave::vec4u;
#pragma unroll
    for (int k = 0; k < V; k++) {
        // volatile: read where it is used, not hoisted out of the row loop
        // (the weights would then sit in registers again).
        const vec4u w = *reinterpret_cast<const volatile vec4u*>(&w_lds[k * 64 + lane]);
        vec4u y;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float l = gfd::bf16::lo(x[k][j]) * scale * gfd::bf16::lo(w[j]);
            const float h = gfd::bf16::hi(x[k][j]) * scale * gfd::bf16::hi(w[j]);
            y[j] = gfd::bf16::pack(l, h);
        }
        gfd::wave::gstore(o + (uint64_t)(k * 64 + lane) * 16, y);
    }
}

template <int V>
__device__ __forceinline__ void rmsnorm_list(const SGListView& view, uint8_t* out, const uint16_t* weight,
                                             float eps, gfd::wave::vec4u* w_lds) {
    // With several compute waves on the list, this one takes entries
    // part, part + parts, ...
    const uint32_t part = view.part, parts = view.parts ? view.parts : 1;
    using gfd::wave::vec4u;
    constexpr uint32_t kRow = (uint32_t)V * 1024;
    const uint32_t lane = (uint32_t)view.lane_id;
#pragma unroll
    for (int k = 0; k < V; k++)
        w_lds[k * 64 + lane] = gfd::wave::gload((uint64_t)(uintptr_t)weight + (uint64_t)(k * 64 + lane) * 16);
    for (uint32_t base = 0; base < view.count; base += 64) {
        uint64_t src = 0;
        uint32_t tag = 0;
        bool ok = false;
        if (base + lane < view.count && (base + lane) % parts == part) {
            const gfd::DeviceSGEntry d = view.get_entry(base + lane);
            ok = d.size == kRow;
            src = d.dst_addr;  // the landed row in HBM
            tag = d.tag;
        }
        for (uint64_t rows = __ballot(ok); rows; rows &= rows - 1) {
            const int j = __builtin_ctzll(rows);
            const uint64_t s0 = __shfl(src, j, 64);
            const uint64_t o0 = (uint64_t)(uintptr_t)out + (uint64_t)(uint32_t)__shfl((int)tag, j, 64) * kRow;
            vec4u x[V];
#pragma unroll
            for (int k = 0; k < V; k++) x[k] = gfd::wave::gload(s0 + (uint64_t)(k * 64 + lane) * 16);
            float ss = sum_squares<V>(x);
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
            store_normalised<V>(x, w_lds, 1.0f / sqrtf(ss / (float)(V * 512) + eps), o0, lane);
        }
    }
}

// The weights, one copy per compute wave: each lane reads back only the
// vectors it stored itself, so no wave waits for another's copy.
__device__ __forceinline__ gfd::wave::vec4u* rms_weights_lds(uint32_t wave_part) {
    __shared__ gfd::wave::vec4u w_lds[gfd::sg_warp_spec::SG_MAX_COMPUTE][14 * 64];
    return w_lds[wave_part < (uint32_t)gfd::sg_warp_spec::SG_MAX_COMPUTE ? wave_part : 0];
}

// One staged row (in LDS) normalised to out + tag * kRow; the slot is handed
// back as soon as the row is in registers.
template <int V>
__device__ __forceinline__ void rmsnorm_staged_row(const gfd::sg_warp_spec::SGRowView& r, uint8_t* out,
                                                   const uint16_t* weight, float eps, gfd::wave::vec4u* w_lds) {
    using gfd::wave::vec4u;
    constexpr uint32_t kRow = (uint32_t)V * 1024;
    const uint32_t lane = (uint32_t)r.lane_id;
    if (r.first) {
#pragma unroll
        for (int k = 0; k < V; k++)
            w_lds[k * 64 + lane] = gfd::wave::gload((uint64_t)(uintptr_t)weight + (uint64_t)(k * 64 + lane) * 16);
    }
    vec4u x[V];
#pragma unroll
    for (int k = 0; k < V; k++) x[k] = r.data[k * 64 + lane];
    r.release();
    float ss = sum_squares<V>(x);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    store_normalised<V>(x, w_lds, 1.0f / sqrtf(ss / (float)(V * 512) + eps),
                        (uint64_t)(uintptr_t)out + (uint64_t)r.tag * kRow, lane);
}

struct RowRMSNorm {
    // Up to SG_MAX_COMPUTE compute waves take the workgroup's rows as the
    // transfer wave stages them in LDS (stage_rows), or share each landed
    // list row by row (list mode).
    static constexpr bool kSharesLists = true;
    static constexpr bool kStagesRows = true;
    uint8_t* out;
    const uint16_t* weight;
    float eps;
    uint32_t row_bytes;
    int stage_rows;
    __device__ uint32_t staged_row_bytes() const { return stage_rows ? row_bytes : 0u; }
    __device__ void row(const gfd::sg_warp_spec::SGRowView& r) const {
        gfd::wave::vec4u* w = rms_weights_lds((uint32_t)gfd::wave::wave_id() - 1);
        switch (row_bytes) {
#define GFD_RMS_CASE(n) \
    case n * 1024: rmsnorm_staged_row<n>(r, out, weight, eps, w); break;
            GFD_RMS_CASE(1) GFD_RMS_CASE(2) GFD_RMS_CASE(3) GFD_RMS_CASE(4) GFD_RMS_CASE(5) GFD_RMS_CASE(6)
            GFD_RMS_CASE(7) GFD_RMS_CASE(8) GFD_RMS_CASE(9) GFD_RMS_CASE(10) GFD_RMS_CASE(11) GFD_RMS_CASE(12)
            GFD_RMS_CASE(13) GFD_RMS_CASE(14)
#undef GFD_RMS_CASE
            default: r.release(); break;
        }
    }
    __device__ void operator()(SGListView v) const {
        gfd::wave::vec4u* w = rms_weights_lds(v.part);
        switch (row_bytes) {
#define GFD_RMS_CASE(n) \
    case n * 1024: rmsnorm_list<n>(v, out, weight, eps, w); break;
            GFD_RMS_CASE(1) GFD_RMS_CASE(2) GFD_RMS_CASE(3) GFD_RMS_CASE(4) GFD_RMS_CASE(5) GFD_RMS_CASE(6)
            GFD_RMS_CASE(7) GFD_RMS_CASE(8) GFD_RMS_CASE(9) GFD_RMS_CASE(10) GFD_RMS_CASE(11) GFD_RMS_CASE(12)
            GFD_RMS_CASE(13) GFD_RMS_CASE(14)
#undef GFD_RMS_CASE
            default: break;
        }
    }
};

struct NoCompute {
    __device__ void operator()(SGListView) const {}
};

struct MoeLists {
    uint64_t host_base, token_stride, dst;
    const int* offsets;
    const int* row_token;
    int num_experts, num_tokens, num_rows;
    uint32_t row_bytes, rows_per_list;
    // The launch's lists and entries fit the ring and the pool
    // (SGWarpSpecSession::gpu_lists_fit): no space or slot waits.
    int fits;
    // Where the lists' headers and entries go: the session's HBM queue
    // (SGDeviceCounters::dev_ring) when they fit, else the host queue.
    gfd::SGTaskQueue* ring;
    // The session's device counters (sg_device_counters of the host queue),
    // so no wave reads the host queue to find them.
    gfd::SGDeviceCounters* cnt;
};

// Submitter wave: posts this workgroup's share of the lists (list L goes to
// workgroup L mod grid); workgroup 0 also tells the transfer waves how many
// lists the launch holds, so that the one landing the last of them ends the
// launch.  Routing entries out of range are reported
// (SG_ERR_BAD_ROW) and become empty entries: nothing outside the host buffer
// is ever read.
__device__ void moe_submit(gfd::SGTaskQueue* sq, const MoeLists& m) {
    using namespace gfd;
    const int lane = wave::lane_id();
    SGDeviceCounters* const cnt = m.cnt;
    // Issued first, beside the offsets' read: the list places depend on them.
    const uint64_t gpu_first =
        __hip_atomic_load(&cnt->list_base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) +
        __hip_atomic_load(&cnt->host_lists, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t entry_first = __hip_atomic_load(&cnt->entry_first, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Lists per expert (one lane per expert, at most 64 experts): `full`
    // lists of rows_per_list rows and at most one shorter one with the rest.
    // Full lists get the first ids (expert-major), the shorter ones the last,
    // longest first, so the lists the transfer waves claim last are the
    // shortest and the end of the launch waits on the least work (longest
    // processing time first).
    int a = 0, b = 0, full = 0, part = 0;
    uint32_t rem = 0;
    if (lane < m.num_experts) {
        a = m.offsets[lane];
        b = m.offsets[lane + 1];
        if (a < 0 || b < a || b > m.num_rows) {
            __hip_atomic_fetch_or(&cnt->error, SG_ERR_BAD_ROW, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            a = b = 0;
        }
        full = (int)((uint32_t)(b - a) / m.rows_per_list);
        rem = (uint32_t)(b - a) % m.rows_per_list;
        part = rem != 0;
    }
    int full_incl = full, part_incl = part;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int tf = __shfl_up(full_incl, o, 64), tp = __shfl_up(part_incl, o, 64);
        if (lane >= o) full_incl += tf, part_incl += tp;
    }
    const int full_excl = full_incl - full;
    // The host's fit check assumed the experts' ranges hold at most num_rows
    // rows together (true for gfd_moe_route's offsets); otherwise wait for
    // space as usual.
    int rows = b - a;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) rows += __shfl_xor(rows, o, 64);
    const bool fits = m.fits && rows <= m.num_rows;
    const uint32_t nfull = (uint32_t)__shfl(full_incl, 63, 64);
    const uint32_t total = nfull + (uint32_t)__shfl(part_incl, 63, 64);
    // Rank of this expert's remainder list among all remainders: longer
    // first, ties in expert order.  Distinct for every expert with one.
    int rank = 0;
    for (int j = 0; j < 64; j++) {
        const uint32_t rj = (uint32_t)__shfl((int)rem, j, 64);
        rank += rj > rem || (rj == rem && j < lane);
    }
    // When the launch's lists fit the ring and the pool, list L sits at ring
    // index gpu_first + L and its entries at pool index entry_first + (rows
    // of the lists before it): the transfer waves, which claim ring indices
    // in order, then take the lists in id order (full lists first, the
    // remainders longest first) whatever order the submitters commit them
    // in.  No submitter ever waits for anything here (no slot is reused, no
    // space is short), so a transfer wave waiting for index gpu_first + L
    // always sees it committed.  Workgroup 0 advances the allocation
    // counters past all of them once, for the host's accounting.
    if (fits && blockIdx.x == 0 && lane == 0) {
        sg::atomic_add_dev(&cnt->list_alloc, total);
        sg::atomic_add_dev(&cnt->entry_alloc, (uint64_t)rows);
    }
    for (uint32_t L = blockIdx.x; L < total; L += gridDim.x) {
        // The expert of list L.  A full list: the highest expert whose first
        // full-list id is <= L.  A remainder: the expert of that rank.
        const bool is_full = L < nfull;
        const uint32_t k = is_full ? L : L - nfull;
        const uint64_t mask = is_full ? __ballot(lane < m.num_experts && (uint32_t)full_excl <= k)
                                      : __ballot(part && (uint32_t)rank == k);
        const int e = is_full ? 63 - __builtin_clzll(mask) : __builtin_ctzll(mask);
        const uint32_t ea = (uint32_t)__shfl(a, e, 64), eb = (uint32_t)__shfl(b, e, 64);
        const uint32_t r0 = is_full ? ea + (k - (uint32_t)__shfl(full_excl, e, 64)) * m.rows_per_list
                                    : eb - (eb - ea) % m.rows_per_list;
        const uint32_t n = min(m.rows_per_list, eb - r0);
        if (!fits && (!sg::sg_wait_entry_space(sq, n) || !sg::sg_wait_list_space(sq))) {
            if (lane == 0) __hip_atomic_fetch_or(&cnt->error, SG_ERR_RING_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        uint64_t pool, slot;
        if (fits) {
            uint32_t before = is_full ? k * m.rows_per_list : nfull * m.rows_per_list;
            if (!is_full) {  // the remainders ranked ahead of this one
                uint32_t mine = part && (uint32_t)rank < k ? rem : 0u;
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) mine += (uint32_t)__shfl_xor((int)mine, o, 64);
                before += mine;
            }
            pool = entry_first + before;
            slot = gpu_first + L;
        } else {
            pool = sg::sg_alloc_entries(sq, n);
            slot = 0;
        }
        if ((uint32_t)lane < n) {
            const uint32_t r = r0 + (uint32_t)lane;
            const int tok = m.row_token[r];
            DeviceSGEntry& d = m.ring->entries[(pool + (uint32_t)lane) % MAX_SG_POOL_ENTRIES];
            d.dst_addr = m.dst + (uint64_t)r * m.row_bytes;
            d.tag = r;
            if (tok >= 0 && tok < m.num_tokens) {
                d.src_addr = m.host_base + (uint64_t)tok * m.token_stride;
                d.size = m.row_bytes;
            } else {
                __hip_atomic_fetch_or(&cnt->error, SG_ERR_BAD_ROW, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                d.src_addr = m.host_base;
                d.size = 0;
            }
        }
        if (!fits) slot = sg::sg_alloc_list(sq);
        if (!sg::sg_commit_list(m.ring, slot, (uint32_t)(pool % MAX_SG_POOL_ENTRIES), n, L, SG_FLAG_NONE, fits))
            break;
    }
    // Host lists queued before the launch land in it too: the transfer wave
    // that lands the last of those and this launch's `total` ends the launch,
    // so stop is raised only once nothing is left to copy, and no wave polls
    // for it meanwhile.  (A list that never lands leaves the transfer waves
    // to the launch's deadline.)
    if (blockIdx.x == 0) sg::sg_stop_when_landed(sq, total, cnt);
}

// Wave 0 transfer, waves 1 .. C compute (C = 1 unless the functor shares
// lists), wave C + 1 submitter, the waves after it transfer helpers.
template <typename F>
__global__ __launch_bounds__(8 * 64) void sg_moe_kernel(gfd::DescriptorQueue* dq, gfd::SGTaskQueue* sq, F fn,
                                                        MoeLists m, int submitter_wave) {
    // (The transfer waves find the counters through sq, one host read per
    // wave as it starts: passing m.cnt here costs the staged-row loop two
    // spilled registers.)
    gfd::sg_warp_spec::_sg_transfer_warp_loop(dq, sq, fn);  // the submitter wave returns from it
    if (gfd::wave::wave_id() == submitter_wave) moe_submit(sq, m);
}

int fail(int code, const char* what) {
    gfd_internal_set_error(what);
    return code ? code : (int)hipErrorInvalidValue;
}

}  // namespace

extern "C" int gfd_sg_session_launch_moe(gfd_sg_session_t s, const void* host_base, uint64_t token_stride,
                                         int num_tokens, const int* offsets, const int* row_token, int num_experts,
                                         int num_rows, uint32_t row_bytes, uint32_t rows_per_list, void* dst,
                                         void* out, const uint16_t* weight, float eps, void* stream) {
    if (!s || !host_base || !offsets || !row_token || !dst || num_tokens <= 0 || num_experts < 1 ||
        num_experts > 64 || num_rows < 0 || num_rows > gfd::MAX_SG_POOL_ENTRIES || row_bytes == 0 ||
        rows_per_list == 0 || rows_per_list > 64 ||
        (out && (!weight || row_bytes % 1024 != 0 || row_bytes > 14 * 1024)))
        return fail(hipErrorInvalidValue, "gfd_sg_session_launch_moe: invalid argument");
    auto* p = static_cast<gfd::SGWarpSpecSession*>(s);
    const int helpers = p->helper_waves();
    // The RMSNorm consumer shares each list between the session's compute
    // waves (num_compute_warps, at most SG_MAX_COMPUTE); transfer only needs one.
    const int compute = out ? std::min(p->compute_waves(), gfd::sg_warp_spec::SG_MAX_COMPUTE) : 1;
    // At most one list more per expert than whole lists of rows.  When they
    // fit the ring and the pool, their headers and entries stay in HBM: the
    // transfer waves read them without a PCIe round trip per list.
    const uint64_t max_lists = (uint64_t)num_experts + (uint64_t)num_rows / rows_per_list;
    if (p->running()) p->synchronize();  // as before_launch would: the ring positions are then current
    const bool fits = p->gpu_lists_fit(max_lists, (uint64_t)num_rows);
    gfd::SGTaskQueue* ring = fits ? p->device_ring() : nullptr;
    if (!ring) ring = p->get_sg_queue();
    p->before_launch(stream, helpers, compute, p->idle_limit_ms(), ring);
    const MoeLists m{(uint64_t)(uintptr_t)host_base, token_stride, (uint64_t)(uintptr_t)dst, offsets, row_token,
                     num_experts, num_tokens, num_rows, row_bytes, rows_per_list, fits ? 1 : 0, ring,
                     gfd::sg_device_counters(p->get_sg_queue())};
    const dim3 grid((unsigned)p->num_blocks()), block((unsigned)(2 + compute + helpers) * 64);
    const char* sr = std::getenv("GFD_SG_STAGED_ROWS");
    const int stage_rows = !(sr && sr[0] == '0');
    if (out)
        hipLaunchKernelGGL(sg_moe_kernel<RowRMSNorm>, grid, block, 0, (hipStream_t)stream, p->get_desc_queue(),
                           p->get_sg_queue(), RowRMSNorm{(uint8_t*)out, weight, eps, row_bytes, stage_rows}, m,
                           1 + compute);
    else
        hipLaunchKernelGGL(sg_moe_kernel<NoCompute>, grid, block, 0, (hipStream_t)stream, p->get_desc_queue(),
                           p->get_sg_queue(), NoCompute{}, m, 2);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(e, "gfd_sg_session_launch_moe: launch failed");
}
