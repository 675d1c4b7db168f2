"""CPU oracle for the scattered host-to-device gather path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this package, and only to verify
results (or, for the CPU baseline, as the thing timed on the host cores).
The product path (``gfd_amd``) never imports it.

What each function restates is cited in ``oracle/oracle.c`` and below.
Pins (tests/test_oracle.py):
  * xorshift64 — Marsaglia's published first outputs for seed 88172645463325252.
  * permutation — is a bijection; brute-force uniformity over all 3! / 4!
    orderings for small n; exact match to an independent pure-Python draw.
  * expected_gather / gather_entries / pool gather — byte equality with a
    naive per-byte loop on tiny inputs, the reference examples' known-answer
    patterns (token i filled with i & 0xFF, examples/02_direct_transfer.cu:50-54;
    floats t*1000+d, examples/01_basic_transfer.cu:138-142; floats i+1,
    test/test_sg_e2e.cu:42), and gap bytes 0xEE never appearing in the output.
  * moe_routing — brute-force top-2 on tiny inputs, tie rule checked on a
    planted tie, list sizes summing to 2*tokens, stability (token order).
  * rmsnorm — closed forms (constant rows, unit weights) and scale invariance.
  * expected_scatter (offload, no reference counterpart) — byte equality with
    a naive per-byte loop on tiny inputs; it inverts expected_gather on the
    tokens' bytes; bytes no token covers keep their value.
  * warp_spec_chunking — the chunk sizes the reference's heuristic gives for
    its documented targets, plus the invariants (power of two, K <= 8, tile
    divisible); warp_spec_expected — brute-force copy on tiny inputs;
    u32_word_checksum — closed forms and a pure-Python loop.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

DATA_SEED = 0x9E3779B97F4A7C15
PERM_SEED = 0xD1B54A32D192ED03
LOGITS_SEED = 0x2545F4914F6CDD1D
GAP_BYTE = 0xEE
MASK64 = (1 << 64) - 1


class SGEntry(ctypes.Structure):
    """Same 24-byte layout as gfd::SGEntry (include/gfd/copy_engine.h:29-33)."""

    _fields_ = [("dst", ctypes.c_uint64), ("src", ctypes.c_void_p), ("size", ctypes.c_size_t)]


_lib = None


def lib():
    """Load liboracle.so, building it with make if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        import subprocess

        subprocess.check_call(["make", "-s", "-C", _HERE])
    L = ctypes.CDLL(_LIB_PATH)
    u64, vp, sz = ctypes.c_uint64, ctypes.c_void_p, ctypes.c_size_t
    L.oracle_xorshift64_next.argtypes = [ctypes.POINTER(u64)]
    L.oracle_xorshift64_next.restype = u64
    L.oracle_xorshift64_fill.argtypes = [u64, vp, sz]
    L.oracle_fill_tokens.argtypes = [vp, sz, sz, sz, u64, ctypes.c_uint8]
    L.oracle_permutation.argtypes = [vp, sz, u64]
    L.oracle_expected_gather.argtypes = [vp, vp, vp, sz, sz, sz]
    L.oracle_expected_scatter.argtypes = [vp, vp, vp, sz, sz, sz]
    L.oracle_gather_entries.argtypes = [vp, vp, ctypes.c_int, u64]
    L.oracle_fnv1a64.argtypes = [vp, sz]
    L.oracle_fnv1a64.restype = u64
    L.oracle_pool_create.argtypes = [ctypes.c_int, vp]
    L.oracle_pool_create.restype = vp
    L.oracle_pool_destroy.argtypes = [vp]
    L.oracle_pool_gather.argtypes = [vp, vp, ctypes.c_int, vp, u64]
    L.oracle_pool_time.argtypes = [vp, vp, ctypes.c_int, vp, u64, ctypes.c_int, vp]
    L.oracle_has_avx512.restype = ctypes.c_int
    _lib = L
    return L


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if isinstance(a, np.ndarray) else a


def xorshift64_seq(seed, n):
    out = np.empty(n, dtype=np.uint64)
    lib().oracle_xorshift64_fill(seed, _ptr(out), n)
    return out


def fill_tokens(region, num_tokens, token_size, stride, seed=DATA_SEED, gap=GAP_BYTE):
    """Fill ``region`` (uint8 ndarray or raw address) with the seeded tokens."""
    if isinstance(region, np.ndarray):
        assert region.dtype == np.uint8 and region.nbytes >= num_tokens * stride
    lib().oracle_fill_tokens(_ptr(region), num_tokens, token_size, stride, seed, gap)


def permutation(n, seed=PERM_SEED):
    perm = np.empty(n, dtype=np.uint32)
    lib().oracle_permutation(_ptr(perm), n, seed)
    return perm


def expected_gather(region, perm, token_size, stride):
    n = len(perm)
    out = np.empty(n * token_size, dtype=np.uint8)
    perm = np.ascontiguousarray(perm, dtype=np.uint32)
    lib().oracle_expected_gather(_ptr(out), _ptr(region), _ptr(perm), n, token_size, stride)
    return out


def expected_scatter(region_before, tokens, perm, token_size, stride):
    """Host region after an offload: token j of ``tokens`` (contiguous, j*T)
    lands at perm[j]*stride; every other byte keeps its value.  No reference
    counterpart (the reference is H2D only)."""
    out = np.array(region_before, dtype=np.uint8, copy=True)
    perm = np.ascontiguousarray(perm, dtype=np.uint32)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint8)
    n = len(perm)
    assert tokens.nbytes >= n * token_size
    if n:
        assert out.nbytes >= int(perm.max()) * stride + token_size
    lib().oracle_expected_scatter(_ptr(out), _ptr(tokens), _ptr(perm), n, token_size, stride)
    return out


def gather_entries(entries, count, out_nbytes, min_dst):
    """Closed form over an SGEntry array: out[e.dst-min_dst+b] = e.src[b]."""
    out = np.zeros(out_nbytes, dtype=np.uint8)
    lib().oracle_gather_entries(_ptr(out), ctypes.cast(entries, ctypes.c_void_p), count, min_dst)
    return out


def fnv1a64(buf):
    buf = np.ascontiguousarray(buf).view(np.uint8)
    return int(lib().oracle_fnv1a64(_ptr(buf), buf.nbytes))


def make_entries(src_base, dst_base, perm, token_size, stride):
    """Entry j: src = src_base + perm[j]*stride, dst = dst_base + j*token_size."""
    n = len(perm)
    arr = (SGEntry * n)()
    a = np.frombuffer(arr, dtype=np.uint64).reshape(n, 3)
    a[:, 0] = np.uint64(dst_base) + np.arange(n, dtype=np.uint64) * np.uint64(token_size)
    a[:, 1] = np.uint64(src_base) + np.asarray(perm, dtype=np.uint64) * np.uint64(stride)
    a[:, 2] = token_size
    return arr


class GatherPool:
    """Restatement of the reference's W-worker ParallelGather
    (src/parallel_gather.cpp:44-116) with persistent spinning workers."""

    def __init__(self, num_workers, cpus=None):
        self.num_workers = num_workers
        cp = None
        if cpus is not None:
            assert len(cpus) == num_workers + 1
            self._cpus = (ctypes.c_int * len(cpus))(*cpus)
            cp = ctypes.cast(self._cpus, ctypes.c_void_p)
        self._h = lib().oracle_pool_create(num_workers, cp)
        if not self._h:
            raise RuntimeError("oracle_pool_create failed")

    def gather(self, entries, count, staging, min_dst):
        lib().oracle_pool_gather(self._h, ctypes.cast(entries, ctypes.c_void_p), count,
                                 _ptr(staging), min_dst)

    def time(self, entries, count, staging, min_dst, iters):
        t = np.empty(iters, dtype=np.float64)
        lib().oracle_pool_time(self._h, ctypes.cast(entries, ctypes.c_void_p), count,
                               _ptr(staging), min_dst, iters, _ptr(t))
        return t

    def close(self):
        if self._h:
            lib().oracle_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


def has_avx512():
    return bool(lib().oracle_has_avx512())


# ----------------------------------------------------------------- MoE (C5)

def moe_logits(num_tokens, num_experts, seed=LOGITS_SEED):
    """Logits [t, e] = ((x >> 40) / 2**24) * 8 - 4 in fp32, x the successive
    xorshift64 outputs in row-major (t, e) order."""
    x = xorshift64_seq(seed, num_tokens * num_experts)
    u = (x >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    return (u * 8.0 - 4.0).astype(np.float32).reshape(num_tokens, num_experts)


def moe_top2(logits):
    """Top-2 experts per token of softmax(logits) == top-2 of logits; ties go
    to the lower expert id.  Returns int32 [T, 2] (best first)."""
    T, E = logits.shape
    # lexicographic sort: larger logit first, then lower expert id
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -logits.astype(np.float64)), axis=1)
    return order[:, :2].astype(np.int32)


def moe_lists(top2, num_experts):
    """Per-expert row lists in token order (stable).  Returns (offsets[E+1],
    token_ids[2T]) with expert-major packing: rows of expert e occupy
    [offsets[e], offsets[e+1]) of the destination."""
    T = top2.shape[0]
    flat_e = top2.reshape(-1)
    flat_t = np.repeat(np.arange(T, dtype=np.int32), 2)
    order = np.argsort(flat_e, kind="stable")
    counts = np.bincount(flat_e, minlength=num_experts)
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    return offsets, flat_t[order]


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x):
    """Round-to-nearest-even fp32 -> bf16 bits (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint16)


def moe_token_values(num_tokens, dim, seed=DATA_SEED):
    """bf16 activations [num_tokens, dim]: successive xorshift64 outputs x ->
    ((x >> 40) / 2**24) * 2 - 1, rounded to bf16 (finite, in [-1, 1])."""
    x = xorshift64_seq(seed, num_tokens * dim)
    u = (x >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    return f32_to_bf16((u * 2.0 - 1.0).astype(np.float32)).reshape(num_tokens, dim)


def moe_weight(dim, seed=PERM_SEED):
    """bf16 RMSNorm weight [dim]: 0.5 + ((x >> 40) / 2**24), rounded to bf16."""
    x = xorshift64_seq(seed, dim)
    u = (x >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    return f32_to_bf16((0.5 + u).astype(np.float32))


def rmsnorm_rows(x_f32, weight_f32, eps):
    """y = x * w / sqrt(mean(x^2) + eps) per row, fp32 (textbook RMSNorm)."""
    x = np.asarray(x_f32, dtype=np.float32)
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    return (x / np.sqrt(ms + eps) * np.asarray(weight_f32, dtype=np.float32)).astype(np.float32)


# ------------------------------------------------------------ sessions

def warp_spec_chunking(token_size, tokens_per_tile=128, tokens_per_chunk=0, double_buffer=False,
                       per_tile_mode=False):
    """(tokens_per_chunk, chunks_per_tile, block threads) of a WarpSpecSession.

    Restates the reference's WarpSpecConfig::effective_tokens_per_chunk
    (include/gfd/warp_spec_session.h:33-52): ~64 KiB chunks for tokens
    <= 512 B, ~256 KiB for tokens >= 64 KiB, else ~128 KiB; at least 4 tokens,
    at most a tile, at most 8 chunks per tile, rounded down to a power of two.
    With 64-lane waves a double-buffered workgroup (1 + 2K waves) stays within
    1024 threads only for K <= 7, so the double-buffer limit is 4 chunks.
    Blocks are 64 * (1 + K) or 64 * (1 + 2K) threads (warp_spec_session.h:59-62
    with 64-lane waves).
    """
    if per_tile_mode:
        c = tokens_per_tile
    elif tokens_per_chunk > 0:
        c = tokens_per_chunk
    else:
        target = 128 * 1024
        if token_size <= 512:
            target = 64 * 1024
        elif token_size >= 65536:
            target = 256 * 1024
        c = max(4, target // token_size)
        c = min(c, tokens_per_tile)
        min_c = tokens_per_tile // (4 if double_buffer else 8)
        if min_c > 0 and c < min_c:
            c = min_c
        p = 1
        while p * 2 <= c:
            p *= 2
        c = p
    k = tokens_per_tile // c
    return c, k, 64 * (1 + (2 * k if double_buffer else k))


def warp_spec_expected(src, dst_before, total_tokens, token_size, tokens_per_tile):
    """Destination after a WarpSpecSession launch: tokens of whole tiles are
    copied from the same offset of src; tokens past the last whole tile are
    untouched (total_tiles = total_tokens / tokens_per_tile,
    include/gfd/warp_spec_session.h:56)."""
    out = np.array(dst_before, dtype=np.uint8, copy=True)
    n = (total_tokens // tokens_per_tile) * tokens_per_tile * token_size
    out[:n] = np.asarray(src, dtype=np.uint8)[:n]
    return out


def u32_word_checksum(buf):
    """Sum (mod 2^64) of buf read as little-endian u32 words, plus the bytes
    of a trailing partial word.  Order-free, so it pins what a consumer wave
    saw of a landed list whatever order its lanes added in."""
    b = np.ascontiguousarray(buf, dtype=np.uint8)
    nw = b.size // 4
    words = b[:nw * 4].view("<u4").astype(np.uint64)
    return (int(words.sum(dtype=np.uint64)) + int(b[nw * 4:].astype(np.uint64).sum())) & MASK64
