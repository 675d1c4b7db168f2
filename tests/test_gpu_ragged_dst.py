"""GPU parity for ragged lists (any entry size, any byte alignment) whose
destinations form one or more runs, the reference's generic path
(src/batch_processor.cpp:726-831, src/direct_submit.cpp:37-145).  Entry sizes
are 1..8999 bytes from seeded random sources in pinned memory; destinations
follow the list order, cut into runs by gaps of odd length, so copies start
and end at every alignment:
  1 run         -> Direct: the zero-copy kernel (about 3 MiB), or, with the
                   kernel route's limit lowered to 1 MiB, the staged gather with
                   one copy per staging chunk and the first 512 KiB of entries
                   moved by the kernel, or the staged gather alone;
                   Queue: staged gather, one copy per staging chunk;
  8 / 40 runs   -> staged gather, one copy per run piece (unaligned pieces);
  100 runs      -> Direct: the zero-copy kernel; Queue: one copy per run.
Every byte of the destination region is compared with the closed form
(sentinel between the runs and after the end)."""
import ctypes
import sys
import time

import numpy as np
import pytest

import gfd_amd

pytestmark = pytest.mark.gpu

SENTINEL = 0xCD
TAIL = 4096
DESC_DTYPE = np.dtype([("src", np.uint64), ("dst", np.uint64), ("size", np.uint32), ("flags", np.uint32),
                       ("user_data", np.uint64), ("sequence", np.uint64), ("_pad", np.uint8, 24)])


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


class RaggedCase:
    """n ragged entries; destinations in list order, cut into nruns runs."""

    def __init__(self, n, nruns, seed, max_size=9000):
        rng = np.random.default_rng(seed)
        self.n = n
        self.sizes = rng.integers(1, max_size, n).astype(np.uint64)
        self.host = gfd_amd.HostBuffer(int(self.sizes.sum()) * 2 + 64)
        self.host.array[:] = rng.integers(0, 256, self.host.nbytes, dtype=np.uint8)
        self.src_offs = np.array([int(rng.integers(0, self.host.nbytes - int(s))) for s in self.sizes], np.uint64)
        gaps = np.zeros(n, np.uint64)
        if nruns > 1:
            cuts = rng.choice(np.arange(1, n), nruns - 1, replace=False)
            gaps[cuts] = rng.integers(0, 2048, nruns - 1) * 2 + 1  # odd: every alignment
        starts = np.concatenate([[0], np.cumsum(self.sizes)[:-1]]).astype(np.uint64) + np.cumsum(gaps)
        self.dst_offs = starts.astype(np.uint64)
        self.region = int(self.dst_offs[-1] + self.sizes[-1])
        self.dst = gfd_amd.DeviceBuffer(self.region + TAIL)
        self.want = np.full(self.region + TAIL, SENTINEL, np.uint8)
        for i in range(n):
            so, do, s = int(self.src_offs[i]), int(self.dst_offs[i]), int(self.sizes[i])
            self.want[do:do + s] = self.host.array[so:so + s]

    def src_addrs(self):
        return np.uint64(self.host.ptr) + self.src_offs

    def dst_addrs(self):
        return np.uint64(self.dst.ptr) + self.dst_offs

    def check(self, what):
        got = self.dst.download()
        bad = np.flatnonzero(got != self.want)
        assert bad.size == 0, "%s: %d mismatched bytes, first at %d" % (what, bad.size, int(bad[0]))
        self.dst.fill(SENTINEL)


@pytest.fixture(scope="module")
def direct_poller():
    p = gfd_amd.CpuPollingThread(None, None, None, 64 << 20, numa_node=-1)
    assert p.init_direct_ce()
    yield p
    p.close()


@pytest.mark.parametrize("nruns,route", [(1, "default"), (1, "staged+head"), (1, "staged"), (8, "default"),
                                         (40, "default"), (100, "default")])
def test_direct_ragged_entries(direct_poller, nruns, route):
    log("submit_direct ragged, %d runs, %s route" % (nruns, route))
    c = RaggedCase(700, nruns, seed=nruns)
    c.dst.fill(SENTINEL)
    entries = (gfd_amd.SGEntry * c.n)()
    a = np.frombuffer(entries, dtype=np.uint64).reshape(c.n, 3)
    a[:, 0] = c.dst_addrs()
    a[:, 1] = c.src_addrs()
    a[:, 2] = c.sizes
    limit = {"default": 8 << 20, "staged+head": 1 << 20, "staged": 0}[route]
    direct_poller.set_direct_zero_copy_max_bytes(limit)
    head = direct_poller.set_direct_zero_copy_head_bytes(512 << 10)
    try:
        for rep in range(2):
            assert direct_poller.submit_direct(entries, c.n) > 0
            c.check("direct, %d runs, %s route, call %d" % (nruns, route, rep))
    finally:
        direct_poller.set_direct_zero_copy_max_bytes(8 << 20)
        direct_poller.set_direct_zero_copy_head_bytes(head)


@pytest.mark.parametrize("n,max_size,route", [(5, 200000, "default"), (3, 100000, "default"),
                                              (40, 70000, "default"), (12, 400000, "staged+head")])
def test_direct_few_large_ragged_entries(direct_poller, n, max_size, route):
    """A short list of large ragged entries is cut into pieces of at least
    4 KiB for the zero-copy kernel's waves (the whole list on the kernel
    route, or the head of a staged list); every byte lands, at every source
    alignment."""
    log("submit_direct few large ragged entries n=%d max=%d %s" % (n, max_size, route))
    c = RaggedCase(n, 1, seed=n, max_size=max_size)
    c.dst.fill(SENTINEL)
    entries = (gfd_amd.SGEntry * c.n)()
    a = np.frombuffer(entries, dtype=np.uint64).reshape(c.n, 3)
    a[:, 0] = c.dst_addrs()
    a[:, 1] = c.src_addrs()
    a[:, 2] = c.sizes
    limit = {"default": 8 << 20, "staged+head": 1 << 20}[route]
    direct_poller.set_direct_zero_copy_max_bytes(limit)
    head = direct_poller.set_direct_zero_copy_head_bytes(512 << 10)
    try:
        for rep in range(2):
            assert direct_poller.submit_direct(entries, c.n) > 0
            c.check("direct, %d entries up to %d B, %s, call %d" % (n, max_size, route, rep))
    finally:
        direct_poller.set_direct_zero_copy_max_bytes(8 << 20)
        direct_poller.set_direct_zero_copy_head_bytes(head)


def queue_ring(q):
    return np.ctypeslib.as_array((ctypes.c_uint8 * (gfd_amd.QUEUE_SIZE * 64)).from_address(q.ptr)).view(DESC_DTYPE)


@pytest.mark.parametrize("nruns", [1, 8, 100])
def test_queue_ragged_entries_cpu_producer(nruns):
    """Queue path, descriptors from a CPU producer: bodies first, then the
    sequence words (x86 stores are seen in program order by the poller)."""
    log("queue ragged, %d runs" % nruns)
    c = RaggedCase(700, nruns, seed=100 + nruns)
    c.dst.fill(SENTINEL)
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, c.dst.ptr, c.host.ptr, c.host.nbytes, numa_node=-1)
    try:
        assert p.init_copy_engine()
        p.start()
        ring = queue_ring(q)
        for rep in range(2):
            base = rep * c.n
            at = (base + np.arange(c.n)) % gfd_amd.QUEUE_SIZE
            flags = np.zeros(c.n, np.uint32)
            flags[-1] = gfd_amd.FLAG_LAST_IN_BATCH
            ring["src"][at] = c.src_addrs()
            ring["dst"][at] = c.dst_addrs()
            ring["size"][at] = c.sizes.astype(np.uint32)
            ring["flags"][at] = flags
            ring["user_data"][at] = np.arange(c.n, dtype=np.uint64)
            ring["sequence"][at] = base + np.arange(c.n, dtype=np.uint64) + 1
            t0 = time.time()
            while q.done_idx < base + c.n:
                assert time.time() - t0 < 20, "done_idx stuck at %d" % q.done_idx
                time.sleep(0.0005)
            c.check("queue, %d runs, round %d" % (nruns, rep))
        assert p.stats()["descriptors_processed"] == 2 * c.n
    finally:
        p.stop()
        p.close()
        q.free()
