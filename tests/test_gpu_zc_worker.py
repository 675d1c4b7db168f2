"""GPU parity of the persistent zero-copy worker (CpuPollingThread::
set_zero_copy_worker; gfd_amd/csrc/zc_worker.cpp, gfd_amd/csrc/aql/
zc_worker.hip): a grid resident on the poller's own AQL queue that copies a
list when the host rings its doorbell.  No reference counterpart: it is a
route of the reference's submit_direct (src/direct_submit.cpp:28-164) and of
its Queue-path batches (src/batch_processor.cpp:605-723), whose contracts
are unchanged: every byte lands before the call returns / before done_idx
passes the batch.  Every destination is compared with the oracle, byte for
byte, and a sentinel tail must survive."""
import ctypes
import sys
import time

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


@pytest.fixture(scope="module")
def worker_poller():
    p = gfd_amd.CpuPollingThread(None, None, None, 16 << 20, numa_node=-1)
    assert p.init_direct_ce()
    p.set_zero_copy_worker(True)
    yield p
    p.close()


def scattered(n, t):
    host = gfd_amd.HostBuffer(n * 2 * t)
    oracle.fill_tokens(host.array, n, t, 2 * t)
    perm = oracle.permutation(n)
    return host, perm, oracle.expected_gather(host.array, perm, t, 2 * t)


# Short lists (below the copy engines' 64 KiB crossover), the config-4 sizes,
# few large tokens that are cut into pieces, sizes that are no multiple of 16,
# an 8 MiB list at the zero-copy route's limit, and 4096 records (64 per copy
# wave, the most a job holds).
@pytest.mark.parametrize("n,t", [(1, 4096), (2, 4096), (16, 4096), (64, 4096), (65, 4096), (256, 4096),
                                 (2048, 512), (2048, 1024), (2048, 2048), (4, 65536), (2, 32768), (3, 1 << 20),
                                 (97, 1000), (5, 12), (2048, 4096), (4096, 256)])
def test_direct_through_the_worker(worker_poller, n, t):
    log("worker direct n=%d t=%d" % (n, t))
    host, perm, want = scattered(n, t)
    dst = gfd_amd.DeviceBuffer(n * t + TAIL)
    entries = gfd_amd.make_entries(np.uint64(host.ptr) + perm.astype(np.uint64) * np.uint64(2 * t), dst.ptr, t)
    for rep in range(3):
        dst.fill(SENTINEL)
        jobs = worker_poller.zero_copy_worker_stats()["jobs"]
        assert worker_poller.submit_direct(entries, n) > 0
        assert worker_poller.zero_copy_worker_stats()["jobs"] == jobs + 1, "not through the worker"
        got = dst.download()
        assert (got[:n * t] == want).all(), "rep %d" % rep
        assert (got[n * t:] == SENTINEL).all()


def test_direct_ragged_and_contiguous_lists_through_the_worker(worker_poller):
    """Entries of 1-20000 bytes at any alignment from random pinned offsets,
    then one contiguous 3 MiB run given as 48 entries (cut into the worker's
    waves), then a single 1 MiB entry."""
    rng = np.random.default_rng(17)
    host = gfd_amd.HostBuffer(8 << 20)
    host.array[:] = rng.integers(0, 256, host.nbytes, dtype=np.uint8)
    dst = gfd_amd.DeviceBuffer((4 << 20) + TAIL)
    lists = []
    sizes = rng.integers(1, 20000, 50)
    srcs = rng.integers(0, host.nbytes - 20000, 50)
    lists.append(("ragged", list(zip(srcs.tolist(), sizes.tolist()))))
    lists.append(("contiguous 48 x 64 KiB", [(1000 + k * 65536, 65536) for k in range(48)]))
    lists.append(("one 1 MiB entry", [(5000, 1 << 20)]))
    for name, ents in lists:
        log("worker direct %s" % name)
        arr = (gfd_amd.SGEntry * len(ents))()
        rec = np.frombuffer(arr, dtype=np.uint64).reshape(-1, 3)  # dst, src, size
        off = 0
        want = np.full(dst.nbytes, SENTINEL, np.uint8)
        for k, (so, n) in enumerate(ents):
            rec[k] = (dst.ptr + off, host.ptr + so, n)
            want[off:off + n] = host.array[so:so + n]
            off += n
        dst.fill(SENTINEL)
        jobs = worker_poller.zero_copy_worker_stats()["jobs"]
        assert worker_poller.submit_direct(arr, len(ents)) > 0
        assert worker_poller.zero_copy_worker_stats()["jobs"] == jobs + 1, name
        assert (dst.download() == want).all(), name


def test_direct_pageable_sources_skip_the_worker(worker_poller):
    n, t = 300, 1000
    log("worker direct, pageable sources")
    region = np.empty(n * 2 * t, np.uint8)
    oracle.fill_tokens(region, n, t, 2 * t)
    perm = oracle.permutation(n)
    dst = gfd_amd.DeviceBuffer(n * t + TAIL)
    dst.fill(SENTINEL)
    entries = gfd_amd.make_entries(region.ctypes.data + perm.astype(np.uint64) * np.uint64(2 * t), dst.ptr, t)
    jobs = worker_poller.zero_copy_worker_stats()["jobs"]
    assert worker_poller.submit_direct(entries, n) > 0
    assert worker_poller.zero_copy_worker_stats()["jobs"] == jobs
    got = dst.download()
    assert (got[:n * t] == oracle.expected_gather(region, perm, t, 2 * t)).all()
    assert (got[n * t:] == SENTINEL).all()


def test_worker_ends_when_idle_and_starts_again(monkeypatch):
    """With a 5 ms idle limit the worker's grid ends between calls 50 ms
    apart; each call dispatches it again, and every byte still lands.  The
    last grid is ended by closing the poller."""
    monkeypatch.setenv("GFD_ZC_WORKER_IDLE_MS", "5")
    n, t = 64, 4096
    host, perm, want = scattered(n, t)
    dst = gfd_amd.DeviceBuffer(n * t + TAIL)
    entries = gfd_amd.make_entries(np.uint64(host.ptr) + perm.astype(np.uint64) * np.uint64(2 * t), dst.ptr, t)
    p = gfd_amd.CpuPollingThread(None, None, None, 1 << 20, numa_node=-1)
    try:
        assert p.init_direct_ce()
        p.set_zero_copy_worker(True)
        for call in range(4):
            log("worker idle exit: call %d" % call)
            dst.fill(SENTINEL)
            assert p.submit_direct(entries, n) > 0
            got = dst.download()
            assert (got[:n * t] == want).all() and (got[n * t:] == SENTINEL).all()
            time.sleep(0.05)
        st = p.zero_copy_worker_stats()
        assert st["jobs"] == 4 and st["launches"] == 4, st
        # Back to back, within the idle limit: one grid serves them all.
        for call in range(5):
            assert p.submit_direct(entries, n) > 0
        st = p.zero_copy_worker_stats()
        assert st["jobs"] == 9 and st["launches"] == 5, st
        got = dst.download()
        assert (got[:n * t] == want).all()
    finally:
        p.close()


@pytest.mark.parametrize("n,t,through_worker", [(2048, 512, True), (2048, 1024, True), (2048, 2048, True),
                                                (300, 1000, True), (1, 4096, True), (9000, 512, True),
                                                (8192, 4096, False)])
def test_queue_batches_through_the_worker(n, t, through_worker):
    """Queue mode with the worker on: GPU-submitted descriptors whose batches
    hold at most 4 MiB are copied by the worker (8192 x 4 KiB batches of 16
    MiB are staged for the copy engines as before); two rounds each, done_idx
    and every byte checked.  9000 x 512 B is 9 batches a round: more jobs than
    the worker's ring of 4, posted while earlier ones run."""
    log("worker queue n=%d t=%d" % (n, t))
    host, perm, want = scattered(n, t)
    src_addrs = np.uint64(host.ptr) + perm.astype(np.uint64) * np.uint64(2 * t)
    dst = gfd_amd.DeviceBuffer(n * t + TAIL)
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, dst.ptr, host.ptr, host.nbytes, numa_node=-1)
    try:
        assert p.init_copy_engine()
        p.set_zero_copy_worker(True)
        p.start()
        tokens = np.zeros((n, 2), np.uint64)
        tokens[:, 0] = src_addrs
        tokens[:, 1] = np.arange(n, dtype=np.uint64)
        dtok = gfd_amd.DeviceBuffer(tokens.nbytes)
        dtok.upload(tokens)
        base = ctypes.c_uint64(0)
        times = np.zeros(1)
        for rep in range(2):
            dst.fill(SENTINEL)
            rc = gfd_amd.lib().gfd_bench_queue(q.ptr, dtok.ptr, dst.ptr, n, t, ctypes.byref(base), 0, 1, 10_000_000,
                                               times.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
            assert rc == 0, gfd_amd.lib().gfd_last_error()
            assert base.value == n * (rep + 1)
            got = dst.download()
            assert (got[:n * t] == want).all(), "round %d" % rep
            assert (got[n * t:] == SENTINEL).all()
        assert q.done_idx == base.value
        jobs, staged = p.zero_copy_worker_stats()["jobs"], p.stats()["staging_batches"]
        if through_worker:
            assert jobs > 0 and staged == 0, (jobs, staged)
        else:
            assert staged > 0, (jobs, staged)  # 16 MiB batches; a short batch cut by a gap may still use the worker
    finally:
        p.stop()
        p.close()
        q.free()
