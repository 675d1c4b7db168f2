"""GPU parity of the wave-specialised sessions (WarpSpecSession,
SGWarpSpecSession) against the oracle: landed bytes are compared byte-exact,
the consumers' results (per-token float sums, per-list u32-word checksums)
exactly.  Cases follow the reference's own tests: test/test_db_small_tiles.cu
(double-buffered tiles, sum = (t+1)*dim), test/test_sg_e2e.cu (one host list
of 4 x 4 KiB floats i+1), test/test_sg_gpu_submit.cu (lists submitted by a
GPU wave)."""
import ctypes
import sys

import numpy as np
import pytest

import gfd_amd
import oracle

pytestmark = pytest.mark.gpu

SENTINEL = 0xCD


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


def auto_helpers(grid):
    """Default helper count: enough for about 32 transfer waves per launch
    (ceil(32 / grid) - 1), at most 3."""
    return max(0, min(3, -(-32 // max(grid, 1)) - 1))


def with_helpers(block, helpers):
    """Workgroup of a session: the reference's block plus this library's
    transfer helper waves (as many as fit in 1024 threads)."""
    h = max(0, min(helpers, (1024 - block) // 64))
    return block + 64 * h, h


def random_host(nbytes, seed):
    h = gfd_amd.HostBuffer(nbytes)
    h.array[:] = np.random.default_rng(seed).integers(0, 256, nbytes, dtype=np.uint8)
    return h


# ------------------------------------------------------------ WarpSpecSession

DB_CASES = [(tc * 32, 32, 16) for tc in (1, 2, 3, 4, 5, 7)] + \
           [(tc * 16, 16, 16) for tc in (1, 2, 3, 5)] + \
           [(tc * 64, 64, 16) for tc in (1, 2, 3)]


@pytest.mark.parametrize("total,tile,chunk", DB_CASES)
def test_warp_spec_db_small_tiles(total, tile, chunk):
    """test/test_db_small_tiles.cu: token t = 256 floats of value t+1,
    double-buffered, grid = min(CUs, tiles); each token's sum is (t+1)*256."""
    log("warp_spec db total=%d tile=%d chunk=%d" % (total, tile, chunk))
    dim = 256
    host = gfd_amd.HostBuffer(total * dim * 4)
    vals = host.array.view(np.float32).reshape(total, dim)
    vals[:] = (np.arange(total, dtype=np.float32) + 1)[:, None]
    dst = gfd_amd.DeviceBuffer(total * dim * 4)
    dst.fill(0)
    sums = gfd_amd.DeviceBuffer(total * 4)
    sums.fill(0)
    res, _ = gfd_amd.warp_spec_run(host.ptr, dst.ptr, total, dim * 4, tile, chunk, double_buffer=True,
                                   num_blocks=total // tile, token_sums=sums.ptr)
    got = sums.download().view(np.float32)
    want = (np.arange(total, dtype=np.float32) + 1) * dim
    assert (got == want).all(), "first bad token %d" % int(np.argmax(got != want))
    assert (dst.download() == host.array).all()
    c, k, block = oracle.warp_spec_chunking(dim * 4, tile, chunk, True)
    assert (res["tokens_per_chunk"], res["chunks_per_tile"]) == (c, k)
    assert (res["block"], res["helper_waves"]) == with_helpers(block, auto_helpers(total // tile))
    assert res["units_done"] == total and res["lists_done"] == total // tile and res["error_bits"] == 0


WS_CASES = [
    # total tokens, token bytes, tile, chunk (0 = auto), double buffer, per-tile mode, blocks (0 = per CU)
    (8192, 4096, 128, 0, False, False, 0),
    (8192, 4096, 128, 0, True, False, 0),
    (1000, 4096, 128, 0, False, False, 0),      # 104 tokens past the last whole tile stay untouched
    (2048, 16384, 128, 0, False, False, 64),
    (512, 65536, 128, 0, True, False, 0),
    (4096, 512, 128, 0, False, False, 0),
    (4096, 1000, 64, 0, False, False, 3),       # token size not a multiple of 16
    (1024, 4096, 128, 0, False, True, 0),       # per-tile mode, K = 1
    (300, 48, 32, 8, True, False, 1),
]


@pytest.mark.parametrize("total,ts,tile,chunk,db,per_tile,blocks", WS_CASES)
def test_warp_spec_parity(total, ts, tile, chunk, db, per_tile, blocks):
    log("warp_spec total=%d ts=%d tile=%d chunk=%d db=%d per_tile=%d blocks=%d" %
        (total, ts, tile, chunk, db, per_tile, blocks))
    host = random_host(total * ts, seed=total * 31 + ts)
    dst = gfd_amd.DeviceBuffer(total * ts + 4096)
    dst.fill(SENTINEL)
    before = dst.download()
    res, times = gfd_amd.warp_spec_run(host.ptr, dst.ptr, total, ts, tile, chunk, db, per_tile, blocks, iters=2)
    got = dst.download()
    want = np.concatenate([oracle.warp_spec_expected(host.array, before[:total * ts], total, ts, tile),
                           before[total * ts:]])
    n_bad = int(np.count_nonzero(got != want))
    assert n_bad == 0, "%d mismatched bytes" % n_bad
    tiles = total // tile
    assert res["lists_done"] == tiles and res["units_done"] == tiles * tile and res["error_bits"] == 0
    c, k, block = oracle.warp_spec_chunking(ts, tile, chunk, db, per_tile)
    assert (res["tokens_per_chunk"], res["chunks_per_tile"]) == (c, k)
    assert (res["block"], res["helper_waves"]) == with_helpers(block, auto_helpers(min(res["grid"], tiles)))
    assert (times > 0).all()


HELPER_CASES = [
    # total tokens, token bytes, tile, chunk, double buffer, per-tile mode
    (1024, 4096, 128, 0, False, True),     # K = 1: a 512 KiB chunk in pieces
    (1024, 4096, 128, 64, True, False),    # K = 2 per slot
    (2048, 1000, 64, 8, False, False),     # K = 8, 8000-byte chunks (one piece each)
    (600, 20000, 32, 32, False, True),     # 640000-byte chunks, not a multiple of 1 KiB
]


@pytest.mark.parametrize("helpers", [0, 1, 3, 6])
@pytest.mark.parametrize("blocks", [1, 8])
@pytest.mark.parametrize("total,ts,tile,chunk,db,per_tile", HELPER_CASES)
def test_warp_spec_helper_waves(total, ts, tile, chunk, db, per_tile, blocks, helpers):
    """Transfer helper waves share each tile's pieces with the transfer wave:
    the landed bytes must not depend on how many there are."""
    log("warp_spec helpers=%d blocks=%d total=%d ts=%d tile=%d chunk=%d db=%d per_tile=%d" %
        (helpers, blocks, total, ts, tile, chunk, db, per_tile))
    host = random_host(total * ts, seed=total + ts + helpers)
    dst = gfd_amd.DeviceBuffer(total * ts + 4096)
    dst.fill(SENTINEL)
    before = dst.download()
    res, _ = gfd_amd.warp_spec_run(host.ptr, dst.ptr, total, ts, tile, chunk, db, per_tile, blocks, iters=2,
                                   helper_waves=helpers)
    want = np.concatenate([oracle.warp_spec_expected(host.array, before[:total * ts], total, ts, tile),
                           before[total * ts:]])
    n_bad = int(np.count_nonzero(dst.download() != want))
    assert n_bad == 0, "%d mismatched bytes" % n_bad
    _, _, block = oracle.warp_spec_chunking(ts, tile, chunk, db, per_tile)
    assert (res["block"], res["helper_waves"]) == with_helpers(block, helpers)
    assert res["lists_done"] == total // tile and res["error_bits"] == 0


def test_warp_spec_helper_waves_token_sums():
    """Compute waves see every piece of their chunk: per-token sums with 3
    helpers splitting one 256 KiB chunk per tile."""
    log("warp_spec helpers token sums")
    total, dim, tile = 2048, 1024, 64
    host = gfd_amd.HostBuffer(total * dim * 4)
    host.array.view(np.float32).reshape(total, dim)[:] = (np.arange(total, dtype=np.float32) + 1)[:, None]
    dst = gfd_amd.DeviceBuffer(total * dim * 4)
    sums = gfd_amd.DeviceBuffer(total * 4)
    sums.fill(0)
    res, _ = gfd_amd.warp_spec_run(host.ptr, dst.ptr, total, dim * 4, tile, 0, False, True, 4, token_sums=sums.ptr,
                                   helper_waves=3)
    want = (np.arange(total, dtype=np.float32) + 1) * dim
    got = sums.download().view(np.float32)
    assert (got == want).all(), "first bad token %d" % int(np.argmax(got != want))
    assert res["helper_waves"] == 3 and res["error_bits"] == 0


def rms_sin_reference(tokens):
    """examples/07_warp_spec_simple.cu:35-58 in float64: per token,
    sum of sin(x r) x r with r = 1/sqrt(mean(x^2) + 1e-6); also the sum of
    the terms' magnitudes, which bounds fp32 rounding."""
    x = tokens.astype(np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=1) + 1e-6)
    y = x * r[:, None]
    terms = np.sin(y) * y
    return terms.sum(axis=1), np.abs(terms).sum(axis=1)


@pytest.mark.parametrize("total,ts,tile,chunk,db,blocks", [(256, 16384, 128, 32, False, 0),
                                                           (256, 16384, 128, 32, True, 0),
                                                           (200, 4100, 64, 16, False, 0), (128, 256, 64, 16, True, 0),
                                                           (1024, 4096, 64, 16, True, 3),
                                                           (1000, 4096, 78, 26, False, 2)])
def test_warp_spec_rms_sin(total, ts, tile, chunk, db, blocks):
    """The RMSNorm + sinf consumer of examples/07_warp_spec_simple.cu through
    WarpSpecSession: every landed token's bytes, and out[t] within fp32
    rounding of a float64 restatement (tolerance 1e-4 of the sum of the
    terms' magnitudes).  Tokens past the last whole tile are not moved and
    their out slots stay untouched.  The consumer lets the framework share a
    chunk's tokens between compute waves (kSplitsChunks); few workgroups
    give each several tiles, so both slots' waves share chunks in steady
    state and at the end, with chunks that do not split evenly into groups."""
    log("warp spec rms+sin total=%d ts=%d tile=%d chunk=%d db=%d blocks=%d" % (total, ts, tile, chunk, db, blocks))
    nf = ts // 4
    host = gfd_amd.HostBuffer(total * ts)
    host.array.view(np.float32)[:] = np.random.default_rng(ts + total).standard_normal(total * nf).astype(np.float32)
    dst = gfd_amd.DeviceBuffer(total * ts)
    dst.fill(0)
    out = gfd_amd.DeviceBuffer(total * 4)
    out.fill(0xCD)
    res, _ = gfd_amd.warp_spec_run_rms_sin(host.ptr, dst.ptr, total, ts, out.ptr, tile, chunk, db, num_blocks=blocks)
    moved = (total // tile) * tile
    assert res["error_bits"] == 0 and res["units_done"] == moved
    assert (dst.download()[:moved * ts] == host.array[:moved * ts]).all()
    got = out.download()
    want, mag = rms_sin_reference(host.array.view(np.float32).reshape(total, nf)[:moved])
    y = got[:moved * 4].view(np.float32).astype(np.float64)
    assert np.all(np.abs(y - want) <= 1e-4 * mag + 1e-6), np.max(np.abs(y - want) / (mag + 1e-30))
    assert (got[moved * 4:] == 0xCD).all()


def test_warp_spec_rejects_oversized_block():
    host = gfd_amd.HostBuffer(4096 * 64)
    dst = gfd_amd.DeviceBuffer(4096 * 64)
    # 16 chunks per tile double-buffered would need 64 * 33 threads
    with pytest.raises(gfd_amd.GfdError):
        gfd_amd.warp_spec_run(host.ptr, dst.ptr, 64, 4096, 64, 4, double_buffer=True)


# --------------------------------------------------------- SGWarpSpecSession

def entries_array(src, dst, size, tag=0):
    return gfd_amd.device_sg_entries(src, dst, size, tag)


def list_checksums(host_bytes, host_base, entries, list_ranges):
    """Expected ListChecksum per list: u32-word checksum of each entry's source bytes."""
    out = {}
    for lid, (a, b) in list_ranges.items():
        s = 0
        for e in entries[a:b]:
            off = int(e["src"]) - host_base
            s += oracle.u32_word_checksum(host_bytes[off:off + int(e["size"])])
        out[lid] = s & oracle.MASK64
    return out


def test_sg_e2e_single_list():
    """test/test_sg_e2e.cu: 4 entries of 4 KiB, floats i+1, one list, one workgroup."""
    log("sg e2e")
    n, t = 4, 4096
    host = gfd_amd.HostBuffer(n * t)
    host.array.view(np.float32)[:] = np.arange(n * t // 4, dtype=np.float32) + 1
    dst = gfd_amd.DeviceBuffer(n * t)
    dst.fill(0)
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=1, idle_limit_ms=5000)
    ent = entries_array(host.ptr + np.arange(n, dtype=np.uint64) * t, dst.ptr + np.arange(n, dtype=np.uint64) * t, t)
    assert s.submit_sg_list(ent, list_id=0) == 0
    s.launch()
    s.synchronize()
    assert (dst.download().view(np.float32) == host.array.view(np.float32)).all()
    st = s.stats()
    assert st["units_done"] == n and st["bytes"] == n * t and st["lists_done"] == 1 and st["error_bits"] == 0
    s.close()


def ragged_lists(rng, host, dst, n_lists, max_entries, max_size):
    """Random lists of random-size entries at random source offsets, disjoint destinations."""
    ents, ranges, off = [], {}, 0
    for lid in range(n_lists):
        k = int(rng.integers(1, max_entries + 1))
        sizes = rng.integers(1, max_size + 1, k)
        srcs = rng.integers(0, host.nbytes - max_size, k)
        a = len(ents)
        for sz, so in zip(sizes, srcs):
            gap = int(rng.integers(0, 33))
            ents.append((host.ptr + int(so), dst.ptr + off + gap, int(sz)))
            off += gap + int(sz)
        ranges[lid] = (a, len(ents))
    assert off <= dst.nbytes
    arr = entries_array([e[0] for e in ents], [e[1] for e in ents], [e[2] for e in ents])
    return arr, ranges


def expected_dst(host, dst_before, dst_ptr, arr):
    out = dst_before.copy()
    for e in arr:
        so, do, n = int(e["src"]) - host.ptr, int(e["dst"]) - dst_ptr, int(e["size"])
        out[do:do + n] = host.array[so:so + n]
    return out


@pytest.mark.parametrize("blocks,compute,helpers", [(1, 1, 3), (8, 1, 3), (0, 1, 3), (0, 3, 3), (1, 1, 0),
                                                    (1, 1, 1), (8, 1, 2), (8, 3, 0)])
def test_sg_ragged_lists_checksum(blocks, compute, helpers):
    log("sg ragged blocks=%d compute=%d helpers=%d" % (blocks, compute, helpers))
    rng = np.random.default_rng(100 + blocks * 7 + compute + 13 * helpers)
    host = random_host(4 << 20, seed=blocks + 11)
    dst = gfd_amd.DeviceBuffer(48 << 20)
    dst.fill(SENTINEL)
    before = dst.download()
    arr, ranges = ragged_lists(rng, host, dst, n_lists=120, max_entries=90, max_size=9000)
    sums = gfd_amd.DeviceBuffer(gfd_amd.MAX_SG_LISTS * 8)
    sums.fill(0)
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=compute, num_blocks=blocks, idle_limit_ms=5000,
                                  helper_waves=helpers)
    for lid, (a, b) in ranges.items():
        s.submit_sg_list(arr[a:b], list_id=lid)
    s.launch(list_sums=sums.ptr)
    s.synchronize()
    assert (dst.download() == expected_dst(host, before, dst.ptr, arr)).all()
    got = sums.download().view(np.uint64)
    want = list_checksums(host.array, host.ptr, arr, ranges)
    for lid, v in want.items():
        assert int(got[lid]) == v, "list %d checksum" % lid
    st = s.stats()
    assert st["units_done"] == len(arr) and st["bytes"] == int(arr["size"].sum()) and st["error_bits"] == 0
    assert st["lists_done"] == len(ranges)
    assert (st["block"], st["helper_waves"]) == (64 * (1 + compute + helpers), helpers)
    s.close()


@pytest.mark.parametrize("blocks,helpers,t", [(0, 0, 4096), (4, 3, 4096), (0, 0, 1000)])
def test_sg_session_offload_lists(blocks, helpers, t):
    """Eviction through the SG session: host-submitted lists whose entries
    copy tokens from HBM (contiguous, token j at j*T) to scattered slots of a
    pinned host region (token j at perm[j]*2T), the reverse of the usual
    direction; no reference counterpart.  Every byte of the region is checked
    against the oracle's offload closed form, the gaps kept."""
    n = 2048
    log("sg offload lists blocks=%d helpers=%d T=%d" % (blocks, helpers, t))
    rng = np.random.default_rng(7 + t)
    toks = rng.integers(0, 256, n * t, dtype=np.uint8)
    src = gfd_amd.DeviceBuffer(n * t)
    src.upload(toks)
    region = gfd_amd.HostBuffer(2 * n * t)
    region.array[:] = SENTINEL
    before = region.array.copy()
    perm = oracle.permutation(n)
    ent = entries_array(src.ptr + np.arange(n, dtype=np.uint64) * np.uint64(t),
                        region.ptr + perm.astype(np.uint64) * np.uint64(2 * t), t)
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=blocks, idle_limit_ms=5000, helper_waves=helpers)
    try:
        for lid in range(16):
            s.submit_sg_list(ent[lid * 128:(lid + 1) * 128], list_id=lid)
        s.launch()
        s.synchronize()
        want = oracle.expected_scatter(before, toks, perm, t, 2 * t)
        assert (region.array == want).all()
        st = s.stats()
        assert st["units_done"] == n and st["bytes"] == n * t and st["lists_done"] == 16 and st["error_bits"] == 0
    finally:
        s.close()


def test_sg_empty_and_tiny_lists_with_helpers():
    """Lists with fewer batches than transfer waves (empty, 1 entry, 65
    entries) keep every helper's acknowledgement in step."""
    log("sg tiny lists helpers")
    rng = np.random.default_rng(77)
    host = random_host(1 << 20, seed=77)
    dst = gfd_amd.DeviceBuffer(4 << 20)
    dst.fill(SENTINEL)
    before = dst.download()
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=2, idle_limit_ms=5000, helper_waves=3)
    sizes = [0, 1, 65, 0, 2, 130, 64, 1]
    ents, off = [], 0
    for lid, k in enumerate(sizes):
        part = []
        for _ in range(k):
            n = int(rng.integers(1, 3000))
            so = int(rng.integers(0, host.nbytes - n))
            part.append((host.ptr + so, dst.ptr + off, n))
            off += n + int(rng.integers(0, 17))
        arr = entries_array([e[0] for e in part], [e[1] for e in part], [e[2] for e in part]) if part else \
            np.zeros(0, dtype=gfd_amd.DEVICE_SG_ENTRY_DTYPE)
        s.submit_sg_list(arr, list_id=lid)
        ents.append(arr)
    s.launch()
    s.synchronize()
    allents = np.concatenate(ents)
    assert (dst.download() == expected_dst(host, before, dst.ptr, allents)).all()
    st = s.stats()
    assert st["lists_done"] == len(sizes) and st["units_done"] == sum(sizes) and st["error_bits"] == 0
    s.close()


@pytest.mark.parametrize("blocks", [1, 8, 16, 64])
def test_sg_default_helper_waves(blocks):
    """Without an explicit count a session adds helpers only to small grids."""
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=blocks, idle_limit_ms=2000)
    st = s.stats()
    assert st["helper_waves"] == auto_helpers(blocks) and st["block"] == 64 * (2 + auto_helpers(blocks))
    s.close()


def test_sg_rejects_too_many_helpers():
    with pytest.raises(gfd_amd.GfdError):
        gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=1, helper_waves=4)


def test_sg_streaming_ring_and_pool_wrap():
    """Lists submitted while the kernel runs: 700 lists (ring of 512) with
    40 entries each (pool of 16384), so both wrap under backpressure."""
    log("sg streaming wrap")
    rng = np.random.default_rng(7)
    t = 1024
    n_lists, epl = 700, 40
    n = n_lists * epl
    host = random_host(n * t, seed=3)
    perm = rng.permutation(n)
    dst = gfd_amd.DeviceBuffer(n * t)
    dst.fill(0)
    arr = entries_array(host.ptr + perm.astype(np.uint64) * t, dst.ptr + np.arange(n, dtype=np.uint64) * t, t)
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=0, idle_limit_ms=5000)
    s.launch()
    for l in range(n_lists):
        s.submit_sg_list(arr[l * epl:(l + 1) * epl], list_id=l % gfd_amd.MAX_SG_LISTS)
    s.synchronize()
    want = host.array.reshape(n, t)[perm].reshape(-1)
    assert (dst.download() == want).all()
    st = s.stats()
    assert st["units_done"] == n and st["lists_done"] == n_lists and st["error_bits"] == 0
    s.close()


def test_sg_relaunch_and_reset():
    """Indices carry over between launches without reset(); reset() restarts them."""
    log("sg relaunch")
    t, n = 2048, 64
    host = random_host(3 * n * t, seed=21)
    dst = gfd_amd.DeviceBuffer(3 * n * t)
    dst.fill(0)
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=4, idle_limit_ms=5000)
    idx = []
    for r in range(3):
        if r == 2:
            s.reset()
        base = r * n
        ent = entries_array(host.ptr + (base + np.arange(n, dtype=np.uint64)) * t,
                            dst.ptr + (base + np.arange(n, dtype=np.uint64)) * t, t)
        idx.append(s.submit_sg_list(ent[: n // 2], list_id=2 * r))
        idx.append(s.submit_sg_list(ent[n // 2:], list_id=2 * r + 1))
        s.launch()
        s.synchronize()
        assert s.stats()["units_done"] == n
    assert idx == [0, 1, 2, 3, 0, 1]
    assert (dst.download() == host.array).all()
    s.close()


def test_sg_submit_without_kernel_rejects_when_ring_full():
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=1, idle_limit_ms=2000)
    host = gfd_amd.HostBuffer(4096)
    dst = gfd_amd.DeviceBuffer(4096)
    ent = entries_array([host.ptr], [dst.ptr], 16)
    for i in range(gfd_amd.MAX_SG_LISTS):
        assert s.submit_sg_list(ent, list_id=i) == i
    with pytest.raises(gfd_amd.GfdError):
        s.submit_sg_list(ent, list_id=0)
    # The queued lists still land once a kernel runs.
    s.launch()
    s.synchronize()
    assert s.stats()["lists_done"] == gfd_amd.MAX_SG_LISTS
    s.close()


@pytest.mark.parametrize("blocks,n_lists,epl,t,helpers", [(1, 4, 8, 4096, 3), (8, 64, 32, 2048, 3),
                                                         (0, 300, 16, 1000, 3), (8, 64, 32, 2048, 0)])
def test_sg_gpu_submit(blocks, n_lists, epl, t, helpers):
    """test/test_sg_gpu_submit.cu: a submitter wave per workgroup builds the
    lists on the GPU (entries from a device table), transfer waves land them,
    the compute wave checksums each list."""
    log("sg gpu submit blocks=%d lists=%d epl=%d t=%d helpers=%d" % (blocks, n_lists, epl, t, helpers))
    n = n_lists * epl
    host = gfd_amd.HostBuffer(n * t)
    if t % 4 == 0:
        host.array.view(np.float32)[:] = np.arange(n * t // 4, dtype=np.float32) + 1
    else:
        host.array[:] = np.random.default_rng(1).integers(0, 256, n * t, dtype=np.uint8)
    dst = gfd_amd.DeviceBuffer(n * t)
    dst.fill(0)
    arr = entries_array(host.ptr + np.arange(n, dtype=np.uint64) * t, dst.ptr + np.arange(n, dtype=np.uint64) * t, t,
                        tag=0)
    d_ent = gfd_amd.DeviceBuffer(arr.nbytes)
    d_ent.upload(arr.view(np.uint8))
    sums = gfd_amd.DeviceBuffer(gfd_amd.MAX_SG_LISTS * 8)
    sums.fill(0)
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=blocks, idle_limit_ms=5000, helper_waves=helpers)
    s.launch_gpu_submit(d_ent.ptr, epl, n_lists, list_sums=sums.ptr)
    s.synchronize(extra_gpu_lists=n_lists)
    assert (dst.download() == host.array).all()
    got = sums.download().view(np.uint64)
    want = list_checksums(host.array, host.ptr, arr, {l: (l * epl, (l + 1) * epl) for l in range(n_lists)})
    for lid, v in want.items():
        assert int(got[lid]) == v, "list %d checksum" % lid
    st = s.stats()
    assert st["lists_done"] == n_lists and st["units_done"] == n and st["error_bits"] == 0
    s.close()


def test_gpu_submit_launch_ends_at_its_deadline_when_a_list_is_withheld():
    """A launch whose lists come from GPU submitters has a deadline (the
    session's idle limit, 2 s here).  The host reserves ring index 0 and never
    commits it, as a host submitter that stopped between allocating and
    committing its list would: the GPU lists queue behind it and none can land.
    The kernel must end by itself at the deadline (the device synchronisation
    returns, in well under the test's limit) with SG_ERR_LIST_WAIT (its
    submitter gave up waiting for the lists) and SG_ERR_DEADLINE (transfer
    waves gave up at the deadline).  After reset() the session works again."""
    import time
    n_lists, epl, t = 8, 16, 4096
    n = n_lists * epl
    log("sg gpu submit with a withheld list, deadline 2 s")
    host = gfd_amd.HostBuffer(n * t)
    host.array[:] = np.random.default_rng(5).integers(0, 256, n * t, dtype=np.uint8)
    dst = gfd_amd.DeviceBuffer(n * t)
    arr = entries_array(host.ptr + np.arange(n, dtype=np.uint64) * t, dst.ptr + np.arange(n, dtype=np.uint64) * t, t)
    d_ent = gfd_amd.DeviceBuffer(arr.nbytes)
    d_ent.upload(arr.view(np.uint8))
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=8, idle_limit_ms=2000, helper_waves=0)
    try:
        alloc = ctypes.c_uint64.from_address(s.queue_ptr() + gfd_amd.SG_QUEUE_LIST_ALLOC_IDX_OFFSET)
        assert alloc.value == 0
        alloc.value = 1  # ring index 0 reserved by the host, never committed
        dst.fill(0)
        t0 = time.monotonic()
        s.launch_gpu_submit(d_ent.ptr, epl, n_lists)
        gfd_amd.synchronize()  # returns once the kernel has ended itself
        elapsed = time.monotonic() - t0
        log("kernel ended after %.2f s" % elapsed)
        with pytest.raises(gfd_amd.GfdError):
            s.synchronize(0)
        st = s.stats()
        assert st["error_bits"] & gfd_amd.SG_ERR_LIST_WAIT, hex(st["error_bits"])
        assert st["error_bits"] & gfd_amd.SG_ERR_DEADLINE, hex(st["error_bits"])
        assert st["lists_done"] == 0
        assert 1.5 < elapsed < 8.0
        s.reset()
        dst.fill(0)
        s.launch_gpu_submit(d_ent.ptr, epl, n_lists)
        s.synchronize(extra_gpu_lists=n_lists)
        assert (dst.download() == host.array).all()
        st = s.stats()
        assert st["lists_done"] == n_lists and st["error_bits"] == 0
    finally:
        s.close()


@pytest.mark.parametrize("blocks,helpers", [(0, 0), (8, 3)])
def test_sg_gpu_submit_offload(blocks, helpers):
    """Eviction lists posted by GPU submitter waves (test/test_sg_gpu_submit.cu's
    pattern with the copy direction reversed; no reference counterpart): 64
    lists of 32 entries, each a 4 KiB token from HBM to its scattered slot in
    a pinned host region.  Every byte of the region against the oracle."""
    n_lists, epl, t = 64, 32, 4096
    n = n_lists * epl
    log("sg gpu submit offload blocks=%d helpers=%d" % (blocks, helpers))
    toks = np.random.default_rng(3).integers(0, 256, n * t, dtype=np.uint8)
    src = gfd_amd.DeviceBuffer(n * t)
    src.upload(toks)
    region = gfd_amd.HostBuffer(2 * n * t)
    region.array[:] = SENTINEL
    before = region.array.copy()
    perm = oracle.permutation(n)
    arr = entries_array(src.ptr + np.arange(n, dtype=np.uint64) * np.uint64(t),
                        region.ptr + perm.astype(np.uint64) * np.uint64(2 * t), t)
    d_ent = gfd_amd.DeviceBuffer(arr.nbytes)
    d_ent.upload(arr.view(np.uint8))
    s = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=blocks, idle_limit_ms=5000, helper_waves=helpers)
    try:
        s.launch_gpu_submit(d_ent.ptr, epl, n_lists)
        s.synchronize(extra_gpu_lists=n_lists)
        assert (region.array == oracle.expected_scatter(before, toks, perm, t, 2 * t)).all()
        st = s.stats()
        assert st["lists_done"] == n_lists and st["units_done"] == n and st["error_bits"] == 0
    finally:
        s.close()
