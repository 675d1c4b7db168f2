"""GPU parity for lists whose destinations are not one contiguous range (the
reference's generic path, src/batch_processor.cpp:726-831): a few destination
runs (packed gather, one copy per run piece), many runs (Direct: the
zero-copy kernel; Queue: per-run copies), pinned and pageable sources.  Every
result is compared byte-exact with the closed form, and bytes between the
destinations must keep their sentinel value."""
import ctypes
import sys
import time

import numpy as np
import pytest

import gfd_amd
import oracle

pytestmark = pytest.mark.gpu

SENTINEL = 0xCD
DESC_DTYPE = np.dtype([("src", np.uint64), ("dst", np.uint64), ("size", np.uint32), ("flags", np.uint32),
                       ("user_data", np.uint64), ("sequence", np.uint64), ("_pad", np.uint8, 24)])


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


@pytest.fixture(scope="module")
def direct_poller():
    p = gfd_amd.CpuPollingThread(None, None, None, 64 << 20, numa_node=-1)
    assert p.init_direct_ce()
    yield p
    p.close()


class Case:
    """n tokens of t bytes at 2t stride (pinned unless pageable), seeded order;
    destination offsets given per entry inside a region of region_bytes."""

    def __init__(self, n, t, dst_offsets, region_bytes, pageable=False):
        self.n, self.t = n, t
        if pageable:
            self.keep = np.empty(n * 2 * t + 4096, np.uint8)
            off = (-self.keep.ctypes.data) % 4096
            self.src_region = self.keep[off:off + n * 2 * t]
            base = self.src_region.ctypes.data
        else:
            self.host = gfd_amd.HostBuffer(n * 2 * t)
            self.src_region = self.host.array
            base = self.host.ptr
        oracle.fill_tokens(self.src_region, n, t, 2 * t)
        self.perm = oracle.permutation(n)
        self.tokens = oracle.expected_gather(self.src_region, self.perm, t, 2 * t).reshape(n, t)
        self.dst = gfd_amd.DeviceBuffer(region_bytes)
        self.dst.fill(SENTINEL)
        self.dst_offsets = np.asarray(dst_offsets, dtype=np.uint64)
        self.src_addrs = np.uint64(base) + self.perm.astype(np.uint64) * np.uint64(2 * t)
        self.entries = (gfd_amd.SGEntry * n)()
        a = np.frombuffer(self.entries, dtype=np.uint64).reshape(n, 3)
        a[:, 0] = np.uint64(self.dst.ptr) + self.dst_offsets
        a[:, 1] = self.src_addrs
        a[:, 2] = t
        self.expect = np.full(region_bytes, SENTINEL, np.uint8)
        for j in range(n):
            o = int(self.dst_offsets[j])
            self.expect[o:o + t] = self.tokens[j]

    def check(self):
        got = self.dst.download()
        bad = int(np.count_nonzero(got != self.expect))
        assert bad == 0, "%d mismatched bytes" % bad


def blocks_layout(n, t, nblocks, gap):
    """Entries in list order fill nblocks contiguous blocks separated by gaps."""
    per = -(-n // nblocks)
    offs = [(j // per) * (per * t + gap) + (j % per) * t for j in range(n)]
    return offs, nblocks * (per * t + gap)


@pytest.mark.parametrize("n,t,nblocks", [(4096, 4096, 10), (2048, 1000, 64), (300, 4096, 2), (8192, 4096, 40)])
def test_direct_few_runs(direct_poller, n, t, nblocks):
    log("direct few runs n=%d t=%d blocks=%d" % (n, t, nblocks))
    offs, region = blocks_layout(n, t, nblocks, 3 * 4096 + 16)
    c = Case(n, t, offs, region)
    for _ in range(2):
        assert direct_poller.submit_direct(c.entries, n) > 0
        c.check()
        c.dst.fill(SENTINEL)


def test_direct_reversed_destinations(direct_poller):
    """A contiguous range written in reverse list order: every entry its own run."""
    log("direct reversed dst")
    n, t = 2048, 4096
    c = Case(n, t, [(n - 1 - j) * t for j in range(n)], n * t)
    assert direct_poller.submit_direct(c.entries, n) > 0
    c.check()


@pytest.mark.parametrize("n,t", [(8192, 4096), (1000, 2048), (512, 65536)])
def test_direct_scattered_pages(direct_poller, n, t):
    """Paged KV cache: n pages scattered over 2n page slots of a device region."""
    log("direct scattered pages n=%d t=%d" % (n, t))
    slots = np.random.default_rng(n + t).permutation(2 * n)[:n]
    c = Case(n, t, slots.astype(np.uint64) * np.uint64(t), 2 * n * t)
    for _ in range(2):
        assert direct_poller.submit_direct(c.entries, n) > 0
        c.check()
        c.dst.fill(SENTINEL)


@pytest.mark.parametrize("scatter", ["pages", "blocks"])
def test_direct_scattered_pageable_sources(direct_poller, scatter):
    log("direct pageable sources, %s" % scatter)
    n, t = 2048, 4096
    if scatter == "pages":
        offs = np.random.default_rng(5).permutation(2 * n)[:n].astype(np.uint64) * np.uint64(t)
        region = 2 * n * t
    else:
        offs, region = blocks_layout(n, t, 8, 4096)
    c = Case(n, t, offs, region, pageable=True)
    assert direct_poller.submit_direct(c.entries, n) > 0
    c.check()


def test_direct_scattered_host_destination_rejected(direct_poller):
    """Destinations outside device memory are refused before anything moves."""
    n, t = 256, 4096
    host_src = gfd_amd.HostBuffer(n * t)
    host_dst = gfd_amd.HostBuffer(2 * n * t)
    entries = (gfd_amd.SGEntry * n)()
    a = np.frombuffer(entries, dtype=np.uint64).reshape(n, 3)
    a[:, 0] = np.uint64(host_dst.ptr) + np.arange(n - 1, -1, -1, dtype=np.uint64) * np.uint64(2 * t)
    a[:, 1] = np.uint64(host_src.ptr) + np.arange(n, dtype=np.uint64) * np.uint64(t)
    a[:, 2] = t
    assert direct_poller.submit_direct(entries, n) < 0


def queue_ring(q):
    return np.ctypeslib.as_array((ctypes.c_uint8 * (gfd_amd.QUEUE_SIZE * 64)).from_address(q.ptr)).view(DESC_DTYPE)


def produce(q, ring, base, c):
    """CPU producer: descriptor bodies first, then the sequence words (x86
    stores are seen in order by the poller)."""
    n = c.n
    slots = (base + np.arange(n)) % gfd_amd.QUEUE_SIZE
    ring["src"][slots] = c.src_addrs
    ring["dst"][slots] = np.uint64(c.dst.ptr) + c.dst_offsets
    ring["size"][slots] = c.t
    flags = np.zeros(n, np.uint32)
    flags[-1] = gfd_amd.FLAG_LAST_IN_BATCH
    ring["flags"][slots] = flags
    ring["user_data"][slots] = np.arange(n, dtype=np.uint64)
    ring["sequence"][slots] = base + np.arange(n, dtype=np.uint64) + 1


@pytest.mark.parametrize("layout", ["blocks", "pages"])
def test_queue_scattered_destinations_cpu_producer(layout):
    """Queue path with descriptors written by a CPU producer: few destination
    runs (staged gather, per-run copies) and scattered pages (per-run copies)."""
    log("queue scattered dst, %s" % layout)
    n, t = 2048, 4096
    if layout == "blocks":
        offs, region = blocks_layout(n, t, 12, 8192)
    else:
        offs = np.random.default_rng(11).permutation(2 * n)[:n].astype(np.uint64) * np.uint64(t)
        region = 2 * n * t
    c = Case(n, t, offs, region)
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, None, None, n * 2 * t, numa_node=-1)
    try:
        assert p.init_copy_engine()
        p.start()
        ring = queue_ring(q)
        for rep in range(2):
            base = rep * n
            produce(q, ring, base, c)
            t0 = time.time()
            while q.done_idx < base + n:
                assert time.time() - t0 < 20, "done_idx stuck at %d" % q.done_idx
                time.sleep(0.0005)
            c.check()
            c.dst.fill(SENTINEL)
        assert q.read_idx == 2 * n
        assert p.stats()["descriptors_processed"] == 2 * n
    finally:
        p.stop()
        p.close()
        q.free()
