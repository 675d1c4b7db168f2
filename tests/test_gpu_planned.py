"""GPU-planned Direct transfer (the reference's
examples/03_gpu_planned_transfer.cu): a kernel selects the tokens routed to
one expert and writes their SG list straight into pinned host memory, then
submit_direct moves them while the poller thread runs.  Known answer as in
the example: token i is filled with i & 0xFF, 4096 tokens routed i % 8,
expert 3 gets 512 tokens (:114-152); every landed byte is checked."""
import ctypes
import sys

import numpy as np
import pytest

import gfd_amd

pytestmark = pytest.mark.gpu

ENTRY_DTYPE = np.dtype([("dst", np.uint64), ("src", np.uint64), ("size", np.uint64)])


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


def plan(routing, expert, cpu_base, stride, gpu_dst, t, cap):
    """Run the planner: routing table in HBM, list and count in pinned host memory."""
    d_routing = gfd_amd.DeviceBuffer(max(routing.nbytes, 4))
    if routing.size:
        d_routing.upload(routing)
    entries = gfd_amd.HostBuffer(max(cap, 1) * ENTRY_DTYPE.itemsize)
    count = gfd_amd.HostBuffer(64)
    count.array.view(np.int32)[0] = -1
    gfd_amd.plan_expert_entries(d_routing.ptr, routing.size, expert, cpu_base, stride, gpu_dst, t, entries.ptr,
                                count.ptr)
    gfd_amd.synchronize()
    n = int(count.array.view(np.int32)[0])
    return entries, n, entries.array.view(ENTRY_DTYPE)[:n].copy()


def test_gpu_planned_direct_transfer_reference_kat():
    log("gpu-planned direct: 4096 tokens, 8 experts, expert 3")
    total, experts, t, target, stride_mul = 4096, 8, 4096, 3, 2
    stride = t * stride_mul
    host = gfd_amd.HostBuffer(total * stride)
    host.array.reshape(total, stride)[:, :t] = (np.arange(total) & 0xFF).astype(np.uint8)[:, None]
    dst = gfd_amd.DeviceBuffer(total // experts * t * 2)
    dst.fill(0)
    routing = (np.arange(total) % experts).astype(np.int32)
    entries, n, got = plan(routing, target, host.ptr, stride, dst.ptr, t, total // experts * 2)
    assert n == total // experts
    toks = np.nonzero(routing == target)[0]
    assert (got["dst"] == np.uint64(dst.ptr) + np.arange(n, dtype=np.uint64) * np.uint64(t)).all()
    assert (got["src"] == np.uint64(host.ptr) + toks.astype(np.uint64) * np.uint64(stride)).all()
    assert (got["size"] == t).all()
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, None, None, dst.nbytes, numa_node=-1)
    try:
        assert p.init_copy_engine() and p.init_direct_ce()
        p.start()  # the example runs Direct beside a started poller
        sg = (gfd_amd.SGEntry * n).from_address(entries.ptr)
        for _ in range(3):
            dst.fill(0)
            assert p.submit_direct(sg, n) > 0
            landed = dst.download()[:n * t].reshape(n, t)
            want = (toks & 0xFF).astype(np.uint8)
            assert (landed == want[:, None]).all(), "slot %d" % int(np.argmax((landed != want[:, None]).any(1)))
            assert (dst.download()[n * t:] == 0).all()
    finally:
        p.stop()
        p.close()
        q.free()


@pytest.mark.parametrize("total,experts", [(1, 1), (1000, 3), (5000, 64), (20000, 7), (1025, 2)])
def test_plan_expert_entries_stable_order(total, experts):
    """Slots follow token order for every expert, including tile edges at
    1024 tokens and experts with no token."""
    log("plan entries total=%d experts=%d" % (total, experts))
    rng = np.random.default_rng(total + experts)
    routing = rng.integers(0, experts, total).astype(np.int32)
    t, stride = 64, 192
    for e in sorted(set([0, experts - 1, experts, int(routing[0])])):
        _, n, got = plan(routing, e, 1 << 40, stride, 1 << 44, t, total)
        toks = np.nonzero(routing == e)[0]
        assert n == len(toks)
        assert (got["src"] == np.uint64(1 << 40) + toks.astype(np.uint64) * np.uint64(stride)).all()
        assert (got["dst"] == np.uint64(1 << 44) + np.arange(n, dtype=np.uint64) * np.uint64(t)).all()


def test_plan_expert_entries_rejects_bad_args():
    buf = gfd_amd.DeviceBuffer(64)
    with pytest.raises(gfd_amd.GfdError):
        gfd_amd.plan_expert_entries(None, 4, 0, 0, 0, 0, 64, buf.ptr, buf.ptr)
    with pytest.raises(gfd_amd.GfdError):
        gfd_amd.plan_expert_entries(buf.ptr, 4, 0, 0, 0, 0, 0, buf.ptr, buf.ptr)
