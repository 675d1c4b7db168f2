"""GPU parity: every gather path of libgfd_amd.so against the oracle,
byte-exact, on seeded scattered layouts (tokens at 2x stride in pinned host
memory, Fisher-Yates order) and the reference examples' known-answer pattern.
Each destination buffer has a sentinel tail that must survive (no overrun)."""
import ctypes
import sys

import numpy as np
import pytest

import gfd_amd
import oracle

pytestmark = pytest.mark.gpu

SENTINEL = 0xCD
TAIL = 4096


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


class Layout:
    def __init__(self, n, t, flags=gfd_amd.HOST_DEFAULT, stride=None):
        self.n, self.t = n, t
        self.stride = stride or 2 * t
        self.host = gfd_amd.HostBuffer(n * self.stride, flags)
        oracle.fill_tokens(self.host.array, n, t, self.stride)
        self.perm = oracle.permutation(n)
        self.expected = oracle.expected_gather(self.host.array, self.perm, t, self.stride)
        self.src_addrs = (np.uint64(self.host.ptr) + self.perm.astype(np.uint64) * np.uint64(self.stride))
        self.dst = gfd_amd.DeviceBuffer(n * t + TAIL)
        self.dst.fill(SENTINEL)

    def check(self):
        got = self.dst.download()
        n_bad = int(np.count_nonzero(got[:self.n * self.t] != self.expected))
        assert n_bad == 0, "%d mismatched bytes" % n_bad
        assert (got[self.n * self.t:] == SENTINEL).all(), "write past the destination range"

    def reset(self):
        self.dst.fill(SENTINEL)


ZC_CASES = [(256, 4096), (8192, 4096), (2048, 65536), (2048, 512), (2048, 1024), (2048, 2048),
            (97, 1000), (3, 48), (1, 16), (5, 12)]


@pytest.mark.parametrize("n,t", ZC_CASES)
def test_zero_copy_tokens_parity(n, t):
    log("zero_copy_tokens n=%d t=%d" % (n, t))
    L = Layout(n, t)
    table = gfd_amd.DeviceBuffer(n * 8)
    table.upload(L.src_addrs)
    gfd_amd.zero_copy_gather_tokens(table.ptr, L.dst.ptr, t, n)
    gfd_amd.synchronize()
    L.check()


# A list of few tokens is cut into pieces for the grid's 64 waves (halving
# each token while twice the pieces fit 64 and the halves stay multiples of 16
# bytes and at least GFD_ZC_MIN_PIECE): 4 x 64 KiB -> 64 pieces of 4 KiB,
# 5 x 24 KiB -> 20 of 6 KiB, 3 x 1 MiB -> 48 of 64 KiB; with a 16-byte floor
# 3 x 4 KiB -> 48 of 256 B and 7 x 64 B -> 28 of 16 B; 1 x 4112 B (257
# vectors), 6 x 8200 B (halves not multiples of 16) and 64 x 64 KiB stay whole.
SPLIT_CASES = [(4, 65536, 4096), (5, 24576, 4096), (3, 1 << 20, 4096), (3, 4096, 16), (7, 64, 16), (1, 4112, 16),
               (6, 8200, 16), (64, 65536, 4096)]


@pytest.mark.parametrize("n,t,min_piece", SPLIT_CASES)
def test_zero_copy_tokens_split_into_pieces(n, t, min_piece, monkeypatch):
    log("zero_copy_tokens pieces n=%d t=%d min_piece=%d" % (n, t, min_piece))
    monkeypatch.setenv("GFD_ZC_MIN_PIECE", str(min_piece))
    L = Layout(n, t)
    table = gfd_amd.DeviceBuffer(n * 8)
    table.upload(L.src_addrs)
    for lds in ("0", "1"):
        monkeypatch.setenv("GFD_ZC_LDS", lds)
        gfd_amd.zero_copy_gather_tokens(table.ptr, L.dst.ptr, t, n)
        gfd_amd.synchronize()
        L.check()
        L.reset()


@pytest.mark.parametrize("n,t,waves,unroll", [(8192, 4096, 0, 4), (2048, 65536, 0, 16), (97, 1000, 0, 8),
                                              (2048, 512, 64, 8), (300, 48, 4, 16)])
def test_zero_copy_lds_staged_parity(n, t, waves, unroll, monkeypatch):
    """The LDS-staged form of the zero-copy kernels (global_load_lds_dwordx4
    into LDS, then LDS -> HBM), selected per call by GFD_ZC_LDS."""
    log("zero_copy LDS-staged n=%d t=%d waves=%d U=%d" % (n, t, waves, unroll))
    monkeypatch.setenv("GFD_ZC_LDS", "1")
    monkeypatch.setenv("GFD_ZC_UNROLL", str(unroll))
    if waves:
        monkeypatch.setenv("GFD_ZC_WAVES", str(waves))
    L = Layout(n, t)
    table = gfd_amd.DeviceBuffer(n * 8)
    table.upload(L.src_addrs)
    gfd_amd.zero_copy_gather_tokens(table.ptr, L.dst.ptr, t, n)
    gfd_amd.synchronize()
    L.check()
    # the generic SG form, same layout
    L.reset()
    entries = gfd_amd.make_entries(L.src_addrs, L.dst.ptr, t)
    dent = gfd_amd.DeviceBuffer(ctypes.sizeof(entries))
    dent.upload(np.frombuffer(entries, dtype=np.uint8))
    gfd_amd.zero_copy_gather(dent.ptr, n)
    gfd_amd.synchronize()
    L.check()


def test_zero_copy_tokens_coherent_source_and_host_table():
    # Fine-grained source and a page table read from pinned host memory.
    log("zero_copy_tokens coherent")
    L = Layout(1024, 4096, flags=gfd_amd.HOST_COHERENT)
    table = gfd_amd.HostBuffer(1024 * 8)
    table.array.view(np.uint64)[:] = L.src_addrs
    gfd_amd.zero_copy_gather_tokens(table.ptr, L.dst.ptr, 4096, 1024)
    gfd_amd.synchronize()
    L.check()


def test_zero_copy_tokens_zero_count_is_noop():
    L = Layout(4, 64)
    gfd_amd.zero_copy_gather_tokens(None, L.dst.ptr, 64, 0)
    gfd_amd.synchronize()
    assert (L.dst.download() == SENTINEL).all()


def _ragged_entries(dst_base, src_base, rng, count, max_size):
    sizes = rng.integers(1, max_size, count)
    src_offs = np.cumsum(np.concatenate([[3], sizes[:-1] * 2 + rng.integers(0, 40, count - 1)]))
    dst_offs = np.cumsum(np.concatenate([[0], sizes[:-1] + rng.integers(0, 24, count - 1)]))
    return sizes, src_offs, dst_offs


# Lists of at most 32 entries are cut into 64 // count slices per entry in the
# kernel (the host does not read the sizes): 5 large entries, one 1 MiB
# entry, 3 tiny ones (empty slices), and 32 entries (2 slices each).
@pytest.mark.parametrize("count,max_size", [(700, 9000), (5, 300000), (1, 1 << 20), (3, 20), (32, 70000)])
@pytest.mark.parametrize("where", ["device", "host"])
def test_zero_copy_sg_generic_ragged(where, count, max_size):
    log("zero_copy_sg ragged (%s entries, %d up to %d B)" % (where, count, max_size))
    rng = np.random.default_rng(11 + count)
    sizes, src_offs, dst_offs = _ragged_entries(0, 0, rng, count, max_size)
    src = gfd_amd.HostBuffer(int(src_offs[-1] + sizes[-1] + 64))
    src.array[:] = rng.integers(0, 256, src.nbytes, dtype=np.uint8)
    dst_len = int(dst_offs[-1] + sizes[-1])
    dst = gfd_amd.DeviceBuffer(dst_len + TAIL)
    dst.fill(SENTINEL)
    entries = (gfd_amd.SGEntry * count)()
    expect = np.full(dst_len + TAIL, SENTINEL, np.uint8)
    for i in range(count):
        entries[i].dst = dst.ptr + int(dst_offs[i])
        entries[i].src = src.ptr + int(src_offs[i])
        entries[i].size = int(sizes[i])
        expect[dst_offs[i]:dst_offs[i] + sizes[i]] = src.array[src_offs[i]:src_offs[i] + sizes[i]]
    raw = np.frombuffer(entries, np.uint8)
    if where == "device":
        tab = gfd_amd.DeviceBuffer(raw.nbytes)
        tab.upload(raw)
    else:
        tab = gfd_amd.HostBuffer(raw.nbytes)
        tab.array[:] = raw
    gfd_amd.zero_copy_gather(tab.ptr, count, None)
    gfd_amd.synchronize()
    assert (dst.download() == expect).all()


def test_zero_copy_sg_matches_tokens_layout():
    log("zero_copy_sg tokens layout")
    L = Layout(2048, 4096)
    entries = gfd_amd.make_entries(L.src_addrs, L.dst.ptr, 4096)
    raw = np.frombuffer(entries, np.uint8)
    tab = gfd_amd.DeviceBuffer(raw.nbytes)
    tab.upload(raw)
    gfd_amd.zero_copy_gather(tab.ptr, 2048, None)
    gfd_amd.synchronize()
    L.check()


# ----------------------------------------------------------- GFD Direct

@pytest.fixture(scope="module")
def direct_poller():
    region = 2048 * 65536 * 2  # largest layout below
    p = gfd_amd.CpuPollingThread(None, None, None, region, numa_node=-1)
    assert p.init_direct_ce()
    log("direct poller: %s" % p.info())
    yield p
    p.close()


DIRECT_CASES = [(256, 4096, 2 << 20), (8192, 4096, 2 << 20), (8192, 4096, 256 << 10), (2048, 65536, 2 << 20),
                (2048, 512, 2 << 20), (2048, 1024, 64 << 10), (2048, 2048, 2 << 20), (97, 1000, 10000),
                (40, 4096, 2 << 20), (4, 65536, 2 << 20), (3, 1 << 20, 2 << 20)]


@pytest.mark.parametrize("route", ["default", "staged"])
@pytest.mark.parametrize("n,t,chunk", DIRECT_CASES)
def test_submit_direct_parity(direct_poller, n, t, chunk, route):
    """Both Direct routes for destination-contiguous lists: by default lists
    up to 8 MiB with pinned sources go through the zero-copy kernel (larger
    ones through staged SDMA copies); 'staged' forces the staged SDMA route
    at every size."""
    log("submit_direct n=%d t=%d chunk=%d route=%s" % (n, t, chunk, route))
    L = Layout(n, t)
    direct_poller.set_direct_chunk_bytes(chunk)
    if route == "staged":
        direct_poller.set_direct_zero_copy_max_bytes(0)
    entries = gfd_amd.make_entries(L.src_addrs, L.dst.ptr, t)
    try:
        for rep in range(2):
            us = direct_poller.submit_direct(entries, n)
            assert us > 0
            L.check()
            L.reset()
    finally:
        direct_poller.set_direct_chunk_bytes(2 << 20)
        direct_poller.set_direct_zero_copy_max_bytes(8 << 20)


@pytest.mark.parametrize("n,t", [(2048, 512), (300, 1000), (2048, 8192), (4096, 3000)])
def test_submit_direct_small_list_from_pageable_sources(direct_poller, n, t):
    """Sources in pageable (not pinned) memory cannot be read by the GPU: a
    small list must take the staged route (gather into pinned staging, then
    SDMA), and a list above the kernel route's limit (16 MiB, 11.7 MiB ragged
    in size) must get no zero-copy head; either way every byte lands."""
    log("submit_direct pageable sources n=%d t=%d" % (n, t))
    region = np.empty(n * 2 * t, np.uint8)
    oracle.fill_tokens(region, n, t, 2 * t)
    perm = oracle.permutation(n)
    dst = gfd_amd.DeviceBuffer(n * t + TAIL)
    dst.fill(SENTINEL)
    entries = gfd_amd.make_entries(region.ctypes.data + perm.astype(np.uint64) * np.uint64(2 * t), dst.ptr, t)
    for rep in range(2):
        assert direct_poller.submit_direct(entries, n) > 0
        got = dst.download()
        assert (got[:n * t] == oracle.expected_gather(region, perm, t, 2 * t)).all()
        assert (got[n * t:] == SENTINEL).all()
        dst.fill(SENTINEL)


def test_submit_direct_head_from_pinned_rest_pageable(direct_poller):
    """A 32 MiB list whose first 1024 tokens are in pinned memory and the
    rest in pageable memory: the zero-copy head takes pinned entries only
    (its check covers the head alone), the gather stages the rest, and every
    byte lands; then the same list with the pinned part moved to the end, so
    the head's sources are pageable and it is refused."""
    n, t, split = 8192, 4096, 1024
    log("submit_direct pinned head + pageable rest n=%d t=%d" % (n, t))
    pinned = gfd_amd.HostBuffer(split * 2 * t)
    pageable = np.empty((n - split) * 2 * t, np.uint8)
    oracle.fill_tokens(pinned.array, split, t, 2 * t)
    oracle.fill_tokens(pageable, n - split, t, 2 * t, seed=0x1234567)
    want = np.concatenate([pinned.array.reshape(split, 2 * t)[:, :t].reshape(-1),
                           pageable.reshape(n - split, 2 * t)[:, :t].reshape(-1)])
    src = np.concatenate([np.uint64(pinned.ptr) + np.arange(split, dtype=np.uint64) * np.uint64(2 * t),
                          np.uint64(pageable.ctypes.data) + np.arange(n - split, dtype=np.uint64) * np.uint64(2 * t)])
    dst = gfd_amd.DeviceBuffer(n * t + TAIL)
    for order in ("pinned first", "pinned last"):
        idx = np.arange(n) if order == "pinned first" else np.roll(np.arange(n), -split)
        entries = gfd_amd.make_entries(src[idx], dst.ptr, t)
        dst.fill(SENTINEL)
        assert direct_poller.submit_direct(entries, n) > 0
        got = dst.download()
        assert (got[:n * t].reshape(n, t) == want.reshape(n, t)[idx]).all(), order
        assert (got[n * t:] == SENTINEL).all()


@pytest.mark.parametrize("n,t", [(16, 4096), (4, 16384), (2, 32768)])
def test_submit_direct_small_list_route(direct_poller, n, t):
    """Lists of at most 64 KiB (the default minimum of the zero-copy route)
    are staged for the copy engines: no kernel launch in the trace.  With the
    minimum at 0 the same list goes through the zero-copy kernel.  Every
    byte lands either way."""
    log("submit_direct small-list route n=%d t=%d" % (n, t))
    L = Layout(n, t)
    entries = gfd_amd.make_entries(L.src_addrs, L.dst.ptr, t)
    prev = direct_poller.set_direct_zero_copy_min_bytes(64 << 10)
    try:
        for zc_min, launches in ((64 << 10, 0), (0, 1)):
            direct_poller.set_direct_zero_copy_min_bytes(zc_min)
            direct_poller.set_trace(True)
            direct_poller.read_trace()
            assert direct_poller.submit_direct(entries, n) > 0
            tr = direct_poller.read_trace()
            direct_poller.set_trace(False)
            assert int(np.count_nonzero(tr["kind"] == 14)) == launches, "min %d" % zc_min
            L.check()
            L.reset()
    finally:
        direct_poller.set_direct_zero_copy_min_bytes(prev)


def test_submit_direct_copy_timeline(direct_poller):
    """The SDMA copy timeline of a Direct call: every copy inside the call's
    window on the copy clock, bytes summing to the gathered bytes."""
    log("submit_direct copy timeline")
    n, t = 8192, 4096
    L = Layout(n, t)
    entries = gfd_amd.make_entries(L.src_addrs, L.dst.ptr, t)
    head = direct_poller.set_direct_zero_copy_head_bytes(0)  # read the setting
    direct_poller.set_direct_zero_copy_head_bytes(head)
    direct_poller.set_copy_timing(True)
    try:
        direct_poller.read_copy_times()  # drop anything recorded before
        t0 = direct_poller.copy_clock_ns()
        assert direct_poller.submit_direct(entries, n) > 0
        t1 = direct_poller.copy_clock_ns()
        c = direct_poller.read_copy_times()
    finally:
        direct_poller.set_copy_timing(False)
    L.check()
    c = c[c["path"] == 1]
    assert len(c) >= 2, "a pipelined 32 MiB gather issues several chunk copies"
    # The zero-copy head (whole tokens) is moved by the kernel, not by SDMA.
    assert int(c["bytes"].sum()) == n * t - (head // t) * t
    assert (c["start_ns"] <= c["end_ns"]).all()
    # Engine timestamps and the host's reading of the same clock can be a
    # fraction of a microsecond apart: allow 2 us at either end of the window.
    assert int(c["start_ns"].min()) >= t0 - 2000 and int(c["end_ns"].max()) <= t1 + 2000
    assert np.all(np.diff(c["seq"].astype(np.int64)) > 0)


def test_submit_direct_concurrent_callers(direct_poller):
    """Two threads calling submit_direct on one poller at once (the reference
    documents the call as thread-safe): calls are serialized, both land."""
    import threading
    log("submit_direct concurrent callers")
    La, Lb = Layout(4096, 4096), Layout(2048, 2048)
    ea = gfd_amd.make_entries(La.src_addrs, La.dst.ptr, La.t)
    eb = gfd_amd.make_entries(Lb.src_addrs, Lb.dst.ptr, Lb.t)
    results = []

    def worker(entries, n, reps):
        for _ in range(reps):
            results.append(direct_poller.submit_direct(entries, n))

    ts = [threading.Thread(target=worker, args=(ea, La.n, 6)), threading.Thread(target=worker, args=(eb, Lb.n, 6))]
    for th in ts:
        th.start()
    for th in ts:
        th.join(timeout=60)
    assert len(results) == 12 and all(r > 0 for r in results)
    La.check()
    Lb.check()


def test_submit_direct_reference_kat(direct_poller):
    # examples/02_direct_transfer.cu:50-54,117-129: token i = i & 0xFF.
    log("submit_direct KAT")
    n, t = 1024, 4096
    host = gfd_amd.HostBuffer(n * 2 * t)
    a = host.array.reshape(n, 2 * t)
    a[:, :t] = (np.arange(n) & 0xFF).astype(np.uint8)[:, None]
    a[:, t:] = oracle.GAP_BYTE
    dst = gfd_amd.DeviceBuffer(n * t)
    srcs = np.uint64(host.ptr) + np.arange(n, dtype=np.uint64) * np.uint64(2 * t)
    entries = gfd_amd.make_entries(srcs, dst.ptr, t)
    assert direct_poller.submit_direct(entries, n) > 0
    assert (dst.download() == np.repeat((np.arange(n) & 0xFF).astype(np.uint8), t)).all()


def test_submit_direct_contiguous_and_scattered_dst(direct_poller):
    log("submit_direct contiguous / scattered dst")
    # fully contiguous source and destination (single split copy)
    host = gfd_amd.HostBuffer(16 << 20)
    host.array[:] = np.random.default_rng(3).integers(0, 256, host.nbytes, dtype=np.uint8)
    dst = gfd_amd.DeviceBuffer(16 << 20)
    n, t = 4096, 4096
    srcs = np.uint64(host.ptr) + np.arange(n, dtype=np.uint64) * np.uint64(t)
    entries = gfd_amd.make_entries(srcs, dst.ptr, t)
    assert direct_poller.submit_direct(entries, n) > 0
    assert (dst.download() == host.array).all()
    # destinations with gaps: one copy per entry
    n2 = 64
    dst2 = gfd_amd.DeviceBuffer(n2 * 2 * t)
    dst2.fill(SENTINEL)
    e2 = (gfd_amd.SGEntry * n2)()
    expect = np.full(n2 * 2 * t, SENTINEL, np.uint8)
    for i in range(n2):
        j = (i * 37) % n2
        e2[i].dst = dst2.ptr + i * 2 * t
        e2[i].src = host.ptr + j * t
        e2[i].size = t
        expect[i * 2 * t:i * 2 * t + t] = host.array[j * t:(j + 1) * t]
    assert direct_poller.submit_direct(e2, n2) > 0
    assert (dst2.download() == expect).all()


def test_submit_direct_rejects_empty(direct_poller):
    assert direct_poller.submit_direct((gfd_amd.SGEntry * 1)(), 0) == -1.0


def test_memcpy_per_token_baseline_parity():
    log("memcpy per token")
    L = Layout(512, 4096)
    t = np.zeros(1)
    rc = gfd_amd.lib().gfd_bench_memcpy_per_token(L.dst.ptr, L.src_addrs.ctypes.data, L.n, L.t, 0, 1,
                                                  t.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    assert rc == 0
    L.check()


# ------------------------------------------------------------- GFD Queue

@pytest.mark.parametrize("n,t", [(2048, 512), (2048, 1024), (2048, 2048), (8192, 4096), (2048, 65536), (1, 4096),
                                 (300, 1000)])
def test_queue_mode_parity(n, t):
    log("queue n=%d t=%d" % (n, t))
    L = Layout(n, t)
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, L.dst.ptr, L.host.ptr, L.host.nbytes, numa_node=-1)
    try:
        assert p.init_copy_engine()
        p.start()
        tokens = np.zeros((n, 2), np.uint64)
        tokens[:, 0] = L.src_addrs
        tokens[:, 1] = np.arange(n, dtype=np.uint64)  # token_id, expert_id = 0
        dtok = gfd_amd.DeviceBuffer(tokens.nbytes)
        dtok.upload(tokens)
        base = ctypes.c_uint64(0)
        times = np.zeros(2)
        for rep in range(2):
            rc = gfd_amd.lib().gfd_bench_queue(q.ptr, dtok.ptr, L.dst.ptr, n, t, ctypes.byref(base), 0, 1,
                                               10_000_000, times.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
            assert rc == 0, gfd_amd.lib().gfd_last_error()
            assert base.value == n * (rep + 1)
            L.check()
            L.reset()
        assert q.done_idx == base.value and q.read_idx == base.value
        s = p.stats()
        assert s["descriptors_processed"] == 2 * n
    finally:
        p.stop()
        p.close()
        q.free()


def _queue_rounds(q, p, L, rounds, base):
    n, t = L.n, L.t
    tokens = np.zeros((n, 2), np.uint64)
    tokens[:, 0] = L.src_addrs
    tokens[:, 1] = np.arange(n, dtype=np.uint64)
    dtok = gfd_amd.DeviceBuffer(tokens.nbytes)
    dtok.upload(tokens)
    b = ctypes.c_uint64(base)
    times = np.zeros(1)
    for _ in range(rounds):
        rc = gfd_amd.lib().gfd_bench_queue(q.ptr, dtok.ptr, L.dst.ptr, n, t, ctypes.byref(b), 0, 1, 10_000_000,
                                           times.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        L.check()
        L.reset()
    return b.value


def test_queue_parity_on_staging_pool_sets():
    """StagingPool (reference include/gfd/staging_pool.h:50-176 and the pool
    branch of src/cpu_polling.cpp:160-245): with a pool of one set sized to
    the region, the first Queue poller takes the set, a second finds it taken
    and allocates its own staging, and once the first is destroyed a third
    takes the set again.  Each moves two rounds of 2048 x 4 KiB, byte-exact."""
    n, t = 2048, 4096
    log("queue on StagingPool sets n=%d t=%d" % (n, t))
    L = Layout(n, t)
    region = L.host.nbytes
    assert gfd_amd.StagingPool.init(1, region, -1)
    qs, ps = [], []
    try:
        for k, want_set in enumerate((0, -1)):
            qs.append(gfd_amd.DescriptorQueue())
            ps.append(gfd_amd.CpuPollingThread(qs[-1], L.dst.ptr, L.host.ptr, region, numa_node=-1))
            assert ps[-1].init_copy_engine()
            info = ps[-1].info()
            assert info["staging_pool_set"] == want_set, info
            assert info["num_staging_buffers"] == 5 and info["staging_buffer_size"] == region
            ps[-1].start()
            assert _queue_rounds(qs[-1], ps[-1], L, 2, 0) == 2 * n
        ps[0].stop()
        ps[0].close()  # releases set 0
        ps[0] = gfd_amd.CpuPollingThread(qs[0], L.dst.ptr, L.host.ptr, region, numa_node=-1)
        assert ps[0].init_copy_engine()
        assert ps[0].info()["staging_pool_set"] == 0, "the released set is taken again"
        ps[0].start()
        assert _queue_rounds(qs[0], ps[0], L, 2, 2 * n) == 4 * n
    finally:
        for p in ps:
            p.stop()
            p.close()
        for q in qs:
            q.free()
        gfd_amd.StagingPool.shutdown()


def test_queue_write_descriptor_safe_through_a_full_ring():
    """write_descriptor_safe (reference include/gfd/device.cuh:120-152) with
    the caller's retry: 3 x QUEUE_SIZE + 100 descriptors of 512 B in one
    launch, so lanes of later laps find their slot still occupied and wait
    for the poller to consume it.  Every byte lands (oracle), done_idx and
    read_idx reach the end, and the ring was full for some lanes.  (With the
    reference's sequence == 0 test a later-lap lane can overwrite a slot
    whose earlier descriptor is not written yet, and the ring stalls; the
    room test here is the poller's read_idx.)"""
    n, t = 3 * gfd_amd.QUEUE_SIZE + 100, 512
    log("queue write_descriptor_safe n=%d t=%d" % (n, t))
    L = Layout(n, t)
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, L.dst.ptr, L.host.ptr, L.host.nbytes, numa_node=-1)
    try:
        assert p.init_copy_engine()
        p.start()
        tokens = np.zeros((n, 2), np.uint64)
        tokens[:, 0] = L.src_addrs
        tokens[:, 1] = np.arange(n, dtype=np.uint64)
        dtok = gfd_amd.DeviceBuffer(tokens.nbytes)
        dtok.upload(tokens)
        status = gfd_amd.HostBuffer(64, gfd_amd.HOST_COHERENT)
        full = gfd_amd.DeviceBuffer(4)
        for rep in range(2):
            full.fill(0)
            status.array.view(np.int32)[:2] = 0
            base = rep * n
            rc = gfd_amd.lib().gfd_queue_submit_tokens_safe(q.ptr, dtok.ptr, L.dst.ptr, n, t, base, 10_000_000,
                                                            status.ptr, full.ptr, None)
            assert rc == 0, gfd_amd.lib().gfd_last_error()
            rc = gfd_amd.lib().gfd_queue_wait(q.ptr, base + n, 10_000_000, status.ptr + 4, None)
            assert rc == 0, gfd_amd.lib().gfd_last_error()
            gfd_amd.synchronize()
            st = status.array.view(np.int32)[:2]
            assert int(st[0]) == 0, "a lane gave up waiting for its slot (round %d)" % rep
            assert int(st[1]) == 0, "done_idx wait timed out (round %d)" % rep
            L.check()
            L.reset()
            hits = int(full.download().view(np.uint32)[0])
            log("  round %d: %d lanes found their slot full" % (rep, hits))
            assert hits > 0, "the ring never filled"
        assert q.done_idx == 2 * n and q.read_idx == 2 * n
    finally:
        p.stop()
        p.close()
        q.free()


@pytest.mark.parametrize("n,t", [(1024, 4096), (3000, 1000), (1, 4096), (16384, 512)])
def test_queue_fused_request_wait_consume(n, t):
    """examples/01_basic_transfer.cu fused kernel: one launch writes the
    descriptors, waits in-kernel for the poller, then reads the landed tokens
    (u32-word checksum per token, exact).  1024 x 4 KiB uses the example's
    floats t*1000+d (:138-142); two rounds move the ring's base slot."""
    log("queue fused n=%d t=%d" % (n, t))
    L = Layout(n, t)
    if (n, t) == (1024, 4096):
        vals = L.host.array.reshape(n, 2, t)[:, 0, :].view(np.float32)
        vals[:] = (np.arange(n, dtype=np.float32)[:, None] * 1000 + np.arange(t // 4, dtype=np.float32)[None, :])
        L.expected = oracle.expected_gather(L.host.array, L.perm, t, L.stride)
    want = [oracle.u32_word_checksum(L.expected[j * t:(j + 1) * t]) for j in range(n)]
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, L.dst.ptr, L.host.ptr, L.host.nbytes, numa_node=-1)
    try:
        assert p.init_copy_engine()
        p.start()
        tokens = np.zeros((n, 2), np.uint64)
        tokens[:, 0] = L.src_addrs
        tokens[:, 1] = np.arange(n, dtype=np.uint64)
        dtok = gfd_amd.DeviceBuffer(tokens.nbytes)
        dtok.upload(tokens)
        sums = gfd_amd.DeviceBuffer(n * 8)
        status = gfd_amd.HostBuffer(64)
        for rep in range(2):
            sums.fill(0)
            status.array.view(np.int32)[0] = 0
            rc = gfd_amd.lib().gfd_queue_fused_checksums(q.ptr, dtok.ptr, L.dst.ptr, n, t, rep * n, 10_000_000,
                                                         sums.ptr, status.ptr, None)
            assert rc == 0, gfd_amd.lib().gfd_last_error()
            gfd_amd.synchronize()
            assert int(status.array.view(np.int32)[0]) == 0, "an in-kernel wait timed out"
            L.check()
            got = sums.download().view(np.uint64)
            bad = [j for j in range(n) if int(got[j]) != want[j]]
            assert not bad, "token %d checksum %d != %d" % (bad[0], int(got[bad[0]]), want[bad[0]])
            L.reset()
        assert q.done_idx == 2 * n
    finally:
        p.stop()
        p.close()
        q.free()
