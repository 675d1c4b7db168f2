// Zero-copy scattered gather for gfx950 (MI355X): wave64 kernels read
// scattered tokens straight out of pinned host memory over PCIe and write them
// contiguously to HBM.  No reference counterpart: the reference always copies
// through CPU staging + copy engines; this is the GPU-initiated alternative
// for the same contract (dst[j*T + b] = token_j[b]).
//
// Memory-level design
//   * A wave takes a batch of up to 64 tokens (entries): lane i loads token
//     i's source address (the KV block / page table entry, normally in HBM)
//     once, and the batch is then copied as one stream of 16-byte vectors
//     (global_load_dwordx4 / global_store_dwordx4) across token boundaries,
//     so a wave covers 1 KiB per instruction and every PCIe read request is
//     a full, contiguous cache-line group.
//   * The copy is branch-free: lanes past the end work on the last vector.
//     A guarded load or store would sit in its own basic block behind a full
//     wait on every earlier memory operation, leaving one request in flight
//     per wave.  With straight-line code a lane keeps U loads in flight.
//   * Grid: a few hundred KiB to 1 MiB of host reads outstanding in total
//     (waves x 64 lanes x U x 16 B) fills the link; far more only queues.
//     The measured optimum is set below (kBytesPerWave ...) and can be
//     overridden with GFD_ZC_WAVES / GFD_ZC_UNROLL (GFD_ZCS_WAVES /
//     GFD_ZCS_UNROLL for the offload kernel, whose posted writes need fewer
//     waves).
//   * Stores are plain 16-byte stores to HBM (coalesced, contiguous).
//   * Staging: in registers by default.  GFD_ZC_LDS=1 selects the form that
//     stages through LDS (global_load_lds_dwordx4 host -> LDS, then LDS ->
//     HBM); measured on MI355X it is within 0.5% of the register form at
//     every size, both being host-link bound.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "gfd/wave_ops.h"

#include "gfd_capi.h"

namespace {

constexpr int kBlock = 256;  // 4 waves
constexpr int kWavesPerBlock = kBlock / 64;
// Waves in flight: one per 128 KiB of the job, between 64 and 256, with 4
// loads in flight per lane (256-1024 KiB of host reads outstanding).
// Measured on MI355X over 64-2048 waves and U = 4/8/16: 8192 x 4 KiB peaks at
// 256 waves (56.8 GB/s) and falls to 52 GB/s at 1024-2048; jobs of 1-4 MiB
// do best at 64 waves; U = 4 is best or within 1% everywhere.
constexpr uint64_t kBytesPerWave = 128 * 1024;
constexpr int kMinWaves = 64, kMaxWaves = 256;
constexpr int kDefaultUnroll = 4;
constexpr int kDefaultLds = 0;
// Offload (HBM -> host): the stores are posted PCIe writes, so few waves fill
// the link.  Measured on MI355X over 16-512 waves and U = 4/8/16: 8192 x 4 KiB
// is flat at 54.8-54.9 GB/s from 16 to 128 waves and 54.5 at 256-512;
// 2048 x 64 KiB peaks at 64 waves (55.5 GB/s).  One wave per 512 KiB, 16-64.
constexpr uint64_t kScatterBytesPerWave = 512 * 1024;
constexpr int kScatterMinWaves = 16, kScatterMaxWaves = 64;
constexpr int kScatterUnroll = 8;
// Smallest piece a token is cut into when a list has too few tokens for its waves.
constexpr int kMinPiece = 4096;

using gfd::wave::BatchLds;
using gfd::wave::GridDone;

// LDS staging area per wave for the staged variant: up to 16 vectors per lane.
constexpr int kStageVecs = 16 * 64;

// Page-table form: token j of num_tokens lives at src_addrs[j] (host) and
// lands at dst + j * token_size.  The unit of work is a piece: each token is
// cut into 2^piece_shift pieces of token_size >> piece_shift bytes (the host
// splits only lists of at most half as many tokens as the waves it targets,
// and only into whole multiples of 16 bytes), so unit u is piece u & (2^s - 1) of
// token u >> s and lands at dst + u * piece.  Wave w copies units
// [w*per_wave, ...) strided over the grid, per_wave <= 64 at a time.
// kLds: stage through LDS.
template <bool kLds>
__global__ __launch_bounds__(kBlock) void zc_gather_tokens(const uint64_t* __restrict__ src_addrs, uint64_t dst,
                                                           uint32_t token_size, uint32_t num_tokens,
                                                           uint32_t piece_shift, uint32_t per_wave, int unroll,
                                                           GridDone done) {
    __shared__ BatchLds lds[kWavesPerBlock];
    __shared__ gfd::wave::vec4u stage[kLds ? kWavesPerBlock : 1][kLds ? kStageVecs : 1];
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint64_t wave = (uint64_t)blockIdx.x * kWavesPerBlock + wid;
    const uint64_t stride = (uint64_t)gridDim.x * kWavesPerBlock * per_wave;
    const uint64_t units = (uint64_t)num_tokens << piece_shift;
    const uint64_t piece = token_size >> piece_shift, piece_mask = (1ull << piece_shift) - 1;
    for (uint64_t first = wave * per_wave; first < units; first += stride) {
        const uint32_t nb = (uint32_t)min((uint64_t)per_wave, units - first);
        uint64_t md = 0, ms = 0, mn = 0;
        if (lane < nb) {
            const uint64_t u = first + lane;
            ms = src_addrs[u >> piece_shift] + (u & piece_mask) * piece;
            md = dst + u * piece;
            mn = piece;
        }
        gfd::wave::copy_batch(unroll, md, ms, mn, nb, &lds[wid], kLds ? stage[wid] : nullptr);
    }
    gfd::wave::signal_grid_done(done, gridDim.x * kWavesPerBlock);
}

// Reverse direction (KV-page offload): token j of num_tokens is read from HBM
// at src + j * token_size and stored to dst_addrs[j] in pinned host memory.
// HBM loads return in ~1-2 us, and the 16-byte stores become posted PCIe
// writes, so each wave moves its batch as one vector stream, exactly as the
// gather does.  Tokens are cut into pieces exactly as in zc_gather_tokens.
template <bool kLds>
__global__ __launch_bounds__(kBlock) void zc_scatter_tokens(const uint64_t* __restrict__ dst_addrs, uint64_t src,
                                                            uint32_t token_size, uint32_t num_tokens,
                                                            uint32_t piece_shift, uint32_t per_wave, int unroll,
                                                            GridDone done) {
    __shared__ BatchLds lds[kWavesPerBlock];
    __shared__ gfd::wave::vec4u stage[kLds ? kWavesPerBlock : 1][kLds ? kStageVecs : 1];
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint64_t wave = (uint64_t)blockIdx.x * kWavesPerBlock + wid;
    const uint64_t stride = (uint64_t)gridDim.x * kWavesPerBlock * per_wave;
    const uint64_t units = (uint64_t)num_tokens << piece_shift;
    const uint64_t piece = token_size >> piece_shift, piece_mask = (1ull << piece_shift) - 1;
    for (uint64_t first = wave * per_wave; first < units; first += stride) {
        const uint32_t nb = (uint32_t)min((uint64_t)per_wave, units - first);
        uint64_t md = 0, ms = 0, mn = 0;
        if (lane < nb) {
            const uint64_t u = first + lane;
            md = dst_addrs[u >> piece_shift] + (u & piece_mask) * piece;
            ms = src + u * piece;
            mn = piece;
        }
        gfd::wave::copy_batch(unroll, md, ms, mn, nb, &lds[wid], kLds ? stage[wid] : nullptr);
    }
    gfd::wave::signal_grid_done(done, gridDim.x * kWavesPerBlock);
}

// Generic SG list: any sizes, any (disjoint) destinations, same batching.
// The sizes are in the table, which the host does not read, so a short list
// is split by count instead: each entry is cut into `pieces` slices of
// ceil(size / pieces) bytes rounded up to 16 (keeping the entry's alignment;
// the last slice takes the rest and slices past the end are empty), and
// unit u is slice u % pieces of entry u / pieces.
template <bool kLds>
__global__ __launch_bounds__(kBlock) void zc_gather_sg(const gfd_sg_entry* __restrict__ entries, uint32_t count,
                                                       uint32_t pieces, uint32_t per_wave, int unroll,
                                                       GridDone done) {
    __shared__ BatchLds lds[kWavesPerBlock];
    __shared__ gfd::wave::vec4u stage[kLds ? kWavesPerBlock : 1][kLds ? kStageVecs : 1];
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint64_t wave = (uint64_t)blockIdx.x * kWavesPerBlock + wid;
    const uint64_t stride = (uint64_t)gridDim.x * kWavesPerBlock * per_wave;
    const uint64_t units = (uint64_t)count * pieces;
    for (uint64_t first = wave * per_wave; first < units; first += stride) {
        const uint32_t nb = (uint32_t)min((uint64_t)per_wave, units - first);
        uint64_t md = 0, ms = 0, mn = 0;
        if (lane < nb) {
            const uint64_t u = first + lane;
            const gfd_sg_entry e = entries[u / pieces];
            const uint64_t step = ((e.size + pieces - 1) / pieces + 15) & ~15ull;
            const uint64_t off = min((u % pieces) * step, e.size);
            md = e.dst + off;
            ms = e.src + off;
            mn = min(step, e.size - off);
        }
        gfd::wave::copy_batch(unroll, md, ms, mn, nb, &lds[wid], kLds ? stage[wid] : nullptr);
    }
    gfd::wave::signal_grid_done(done, gridDim.x * kWavesPerBlock);
}

int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

// Launch shape for n entries: (blocks, entries per wave, unroll).
struct Shape {
    uint32_t blocks, per_wave;
    uint32_t piece_shift;  // tokens cut into 2^piece_shift pieces
    int unroll;
    bool lds;  // stage through LDS
};

struct ShapeDefaults {
    uint64_t bytes_per_wave;
    int min_waves, max_waves, unroll;
    const char* waves_env;
    const char* unroll_env;
};
constexpr ShapeDefaults kGatherShape{kBytesPerWave, kMinWaves, kMaxWaves, kDefaultUnroll, "GFD_ZC_WAVES",
                                     "GFD_ZC_UNROLL"};
constexpr ShapeDefaults kScatterShape{kScatterBytesPerWave, kScatterMinWaves, kScatterMaxWaves, kScatterUnroll,
                                      "GFD_ZCS_WAVES", "GFD_ZCS_UNROLL"};

// n entries of total_bytes.  token_size != 0: the entries are tokens of that
// size, which may be cut into pieces: a list of fewer tokens than the target
// number of waves would leave waves idle and give each busy wave a whole large
// token to stream on its own (4 x 64 KiB on 4 waves ran at 7 GB/s).  Tokens
// are then halved while twice the units still fit the target, the halves stay
// whole multiples of 16 bytes and at least GFD_ZC_MIN_PIECE bytes (4 KiB: one
// pass of a wave at 4 loads per lane), so every unit gets a wave of its own.
// Lists of more than half the target in tokens are never cut.
Shape shape_for(uint64_t n, uint64_t total_bytes, const ShapeDefaults& d = kGatherShape, uint32_t token_size = 0) {
    // Read per call (a getenv is ~100 ns against a launch of microseconds),
    // so a process can sweep launch shapes.
    const int dflt = (int)std::min<uint64_t>(
        std::max<uint64_t>(total_bytes / d.bytes_per_wave, (uint64_t)d.min_waves), (uint64_t)d.max_waves);
    const int target = std::max(4, env_int(d.waves_env, dflt));
    const int unroll_env = env_int(d.unroll_env, d.unroll);
    uint32_t shift = 0;
    if (token_size != 0) {
        const uint64_t min_piece = (uint64_t)std::max(16, env_int("GFD_ZC_MIN_PIECE", kMinPiece));
        while ((n << (shift + 1)) <= (uint64_t)target && shift < 16) {
            const uint64_t half = (uint64_t)token_size >> (shift + 1);
            if (half < min_piece || (half & 15) != 0 || (half << (shift + 1)) != token_size) break;
            shift++;
        }
    }
    n <<= shift;
    uint64_t per_wave = (n + target - 1) / target;
    per_wave = std::min<uint64_t>(std::max<uint64_t>(per_wave, 1), 64);
    const uint64_t waves = (n + per_wave - 1) / per_wave;
    Shape s;
    s.per_wave = (uint32_t)per_wave;
    s.piece_shift = shift;
    s.blocks = (uint32_t)((waves + kWavesPerBlock - 1) / kWavesPerBlock);
    s.unroll = unroll_env >= 16 ? 16 : (unroll_env >= 8 ? 8 : 4);
    s.lds = env_int("GFD_ZC_LDS", kDefaultLds) != 0;
    return s;
}

// Launchers; `done` is {nullptr, nullptr, 0} for stream-ordered completion.
int launch_gather_tokens(const uint64_t* src_addrs, void* dst, uint32_t token_size, int num_tokens, void* stream,
                         GridDone done) {
    if (num_tokens < 0 || (num_tokens > 0 && (!src_addrs || !dst || token_size == 0)))
        return (int)hipErrorInvalidValue;
    if (num_tokens == 0) return 0;
    if ((uint64_t)token_size >= (1ull << 30)) return (int)hipErrorInvalidValue;  // 1 GiB per token at most
    const Shape s = shape_for((uint64_t)num_tokens, (uint64_t)num_tokens * token_size, kGatherShape, token_size);
    if (s.lds)
        hipLaunchKernelGGL(zc_gather_tokens<true>, dim3(s.blocks), dim3(kBlock), 0, (hipStream_t)stream, src_addrs,
                           (uint64_t)(uintptr_t)dst, token_size, (uint32_t)num_tokens, s.piece_shift, s.per_wave,
                           s.unroll, done);
    else
        hipLaunchKernelGGL(zc_gather_tokens<false>, dim3(s.blocks), dim3(kBlock), 0, (hipStream_t)stream, src_addrs,
                           (uint64_t)(uintptr_t)dst, token_size, (uint32_t)num_tokens, s.piece_shift, s.per_wave,
                           s.unroll, done);
    return (int)hipGetLastError();
}

int launch_scatter_tokens(const uint64_t* dst_addrs, const void* src, uint32_t token_size, int num_tokens,
                          void* stream, GridDone done) {
    if (num_tokens < 0 || (num_tokens > 0 && (!dst_addrs || !src || token_size == 0)))
        return (int)hipErrorInvalidValue;
    if (num_tokens == 0) return 0;
    if ((uint64_t)token_size >= (1ull << 30)) return (int)hipErrorInvalidValue;  // 1 GiB per token at most
    const Shape s = shape_for((uint64_t)num_tokens, (uint64_t)num_tokens * token_size, kScatterShape, token_size);
    if (s.lds)
        hipLaunchKernelGGL(zc_scatter_tokens<true>, dim3(s.blocks), dim3(kBlock), 0, (hipStream_t)stream, dst_addrs,
                           (uint64_t)(uintptr_t)src, token_size, (uint32_t)num_tokens, s.piece_shift, s.per_wave,
                           s.unroll, done);
    else
        hipLaunchKernelGGL(zc_scatter_tokens<false>, dim3(s.blocks), dim3(kBlock), 0, (hipStream_t)stream, dst_addrs,
                           (uint64_t)(uintptr_t)src, token_size, (uint32_t)num_tokens, s.piece_shift, s.per_wave,
                           s.unroll, done);
    return (int)hipGetLastError();
}

// Waves a short list is aimed at (GFD_ZC_WAVES, else the minimum grid).
int short_list_waves() { return std::max(4, env_int(kGatherShape.waves_env, kGatherShape.min_waves)); }

// slice: the table is the caller's list as it is, so a list of at most half
// the target waves' entries gets target / count waves per entry (slices of a
// small entry may be empty).  Without it, each record is one wave's work (the
// caller has cut the list into pieces already).
int launch_gather_sg(const gfd_sg_entry* entries, int count, void* stream, GridDone done, bool slice = true) {
    if (count < 0 || (count > 0 && !entries)) return (int)hipErrorInvalidValue;
    if (count == 0) return 0;
    // Sizes are in the entry table, not known here: shape for 4 KiB entries.
    const int target = short_list_waves();
    const uint32_t pieces = slice && 2 * count <= target ? (uint32_t)(target / count) : 1u;
    const Shape s = shape_for((uint64_t)count * pieces, (uint64_t)count * pieces * 4096);
    if (s.lds)
        hipLaunchKernelGGL(zc_gather_sg<true>, dim3(s.blocks), dim3(kBlock), 0, (hipStream_t)stream, entries,
                           (uint32_t)count, pieces, s.per_wave, s.unroll, done);
    else
        hipLaunchKernelGGL(zc_gather_sg<false>, dim3(s.blocks), dim3(kBlock), 0, (hipStream_t)stream, entries,
                           (uint32_t)count, pieces, s.per_wave, s.unroll, done);
    return (int)hipGetLastError();
}

GridDone grid_done(unsigned int* counter, uint64_t* host_word, uint64_t value) { return GridDone{counter, host_word, value}; }

}  // namespace

extern "C" int gfd_zero_copy_gather_tokens(const uint64_t* src_addrs, void* dst, uint32_t token_size,
                                           int num_tokens, void* stream) {
    return launch_gather_tokens(src_addrs, dst, token_size, num_tokens, stream, GridDone{nullptr, nullptr, 0});
}

extern "C" int gfd_zero_copy_scatter_tokens(const uint64_t* dst_addrs, const void* src, uint32_t token_size,
                                            int num_tokens, void* stream) {
    return launch_scatter_tokens(dst_addrs, src, token_size, num_tokens, stream, GridDone{nullptr, nullptr, 0});
}

extern "C" int gfd_zero_copy_gather(const gfd_sg_entry* entries, int count, void* stream) {
    return launch_gather_sg(entries, count, stream, GridDone{nullptr, nullptr, 0});
}

extern "C" int gfd_zero_copy_gather_tokens_signal(const uint64_t* src_addrs, void* dst, uint32_t token_size,
                                                  int num_tokens, unsigned int* done_counter, uint64_t* done_word,
                                                  uint64_t done_value, void* stream) {
    if (!done_counter || !done_word) return (int)hipErrorInvalidValue;
    return launch_gather_tokens(src_addrs, dst, token_size, num_tokens, stream,
                                grid_done(done_counter, done_word, done_value));
}

extern "C" int gfd_zero_copy_scatter_tokens_signal(const uint64_t* dst_addrs, const void* src, uint32_t token_size,
                                                   int num_tokens, unsigned int* done_counter, uint64_t* done_word,
                                                   uint64_t done_value, void* stream) {
    if (!done_counter || !done_word) return (int)hipErrorInvalidValue;
    return launch_scatter_tokens(dst_addrs, src, token_size, num_tokens, stream,
                                 grid_done(done_counter, done_word, done_value));
}

extern "C" int gfd_zero_copy_gather_signal(const gfd_sg_entry* entries, int count, unsigned int* done_counter,
                                           uint64_t* done_word, uint64_t done_value, void* stream) {
    if (!done_counter || !done_word) return (int)hipErrorInvalidValue;
    return launch_gather_sg(entries, count, stream, grid_done(done_counter, done_word, done_value));
}

extern "C" int gfd_zero_copy_gather_signal_presliced(const gfd_sg_entry* entries, int count,
                                                     unsigned int* done_counter, uint64_t* done_word,
                                                     uint64_t done_value, void* stream) {
    if (!done_counter || !done_word) return (int)hipErrorInvalidValue;
    return launch_gather_sg(entries, count, stream, grid_done(done_counter, done_word, done_value), false);
}

extern "C" int gfd_zero_copy_target_waves(void) { return short_list_waves(); }
