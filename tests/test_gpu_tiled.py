"""GPU parity of the CPU poller's tiled mode (the reference's per-tile
baseline, examples/07_warp_spec_simple.cu:88-134 and :342-418): a kernel
claims ring slots with the tiled device primitives, submits each tile chunk
by chunk (or whole), and waits on the tile's progress word, which the poller
raises after its copies (copy-engine writes into HBM, or host-memory words).
The landed tokens are compared byte-exact with the source, each token's
u32-word checksum read by the kernel exactly, and every tile's progress word
must equal tokens_per_tile.  Two rounds per case, resetting as the example
does (stop, reset queue and progress, reset_stats, launch, start)."""
import sys

import numpy as np
import pytest

import gfd_amd
import oracle

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


@pytest.mark.parametrize("tiles,T,C,ts,whole,dev_signals", [
    (8, 128, 32, 4096, False, True),     # the example's shape: 4 chunks per tile
    (8, 128, 32, 4096, True, True),      # submit_tile: one claim per tile
    (16, 64, 64, 1000, False, True),     # one chunk per tile, tokens not a multiple of 16
    (4, 256, 16, 2048, False, False),    # progress words in host memory
    (100, 32, 8, 512, False, True),      # many small tiles in flight at once
])
def test_tiled_poller_mode(tiles, T, C, ts, whole, dev_signals):
    log("tiled poller tiles=%d T=%d C=%d ts=%d whole=%d dev=%d" % (tiles, T, C, ts, whole, dev_signals))
    n = tiles * T
    host = gfd_amd.HostBuffer(n * ts)
    host.array[:] = np.random.default_rng(n + ts).integers(0, 256, n * ts, dtype=np.uint8)
    want = [oracle.u32_word_checksum(host.array[g * ts:(g + 1) * ts]) for g in range(n)]
    dst = gfd_amd.DeviceBuffer(n * ts + 4096)
    sums = gfd_amd.DeviceBuffer(n * 8)
    status = gfd_amd.HostBuffer(64)
    tq = gfd_amd.TiledQueue(tiles, T, C, ts, device_signals=dev_signals)
    p = gfd_amd.CpuPollingThread(tq, dst.ptr, host.ptr, host.nbytes, numa_node=-1)
    try:
        p.set_tiled_queue(tq)
        assert p.init_copy_engine()
        for rnd in range(2):
            p.stop()
            tq.reset()
            p.reset_stats()
            dst.fill(0xCD)
            sums.fill(0)
            status.array.view(np.int32)[0] = 0
            gfd_amd.tiled_poller_run(tq, host.ptr, dst.ptr, sums.ptr, status.ptr, whole_tile=whole)
            p.start()
            gfd_amd.synchronize()
            assert int(status.array.view(np.int32)[0]) == 0, "a tile wait timed out (round %d)" % rnd
            got = dst.download()
            assert (got[:n * ts] == host.array).all(), "landed bytes differ (round %d)" % rnd
            assert (got[n * ts:] == 0xCD).all()
            s = sums.download().view(np.uint64)
            bad = [g for g in range(n) if int(s[g]) != want[g]]
            assert not bad, "token %d checksum (round %d)" % (bad[0], rnd)
            assert (tq.tile_progress() == T).all()
            assert p.stats()["descriptors_processed"] == n
    finally:
        p.stop()
        p.close()
        tq.free()


def test_tiled_poller_run_rejects_launch_larger_than_ring():
    tq = gfd_amd.TiledQueue(1024, 32, 32, 64)  # 32768 slots > QUEUE_SIZE
    buf = gfd_amd.DeviceBuffer(64)
    st = gfd_amd.HostBuffer(64)
    try:
        with pytest.raises(gfd_amd.GfdError):
            gfd_amd.tiled_poller_run(tq, buf.ptr, buf.ptr, buf.ptr, st.ptr)
    finally:
        tq.free()
