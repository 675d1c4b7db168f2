"""GPU parity of the offload path (HBM -> pinned host, the reverse of the
gather; no reference counterpart, docs/Architecture.md:642,993 lists D2H as
future work): the zero-copy scatter kernel and the direction-agnostic SG
kernel against the oracle's closed form, byte-exact.  Host regions are
pre-filled with a sentinel that must survive wherever no token lands; at full
sizes a gather -> offload round trip must restore the host region exactly."""
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


class Offload:
    """n tokens of t bytes contiguous in HBM, offloaded to host slots
    perm[j] * stride of a pinned region (2x stride: every other slot is a gap)."""

    def __init__(self, n, t, stride=None, flags=gfd_amd.HOST_DEFAULT, seed=0):
        self.n, self.t = n, t
        self.stride = stride or 2 * t
        self.tokens = np.random.default_rng(seed + n * 31 + t).integers(0, 256, n * t, dtype=np.uint8)
        self.src = gfd_amd.DeviceBuffer(max(n * t, 1))
        if n:
            self.src.upload(self.tokens)
        self.host = gfd_amd.HostBuffer(max(n * self.stride, 16), flags)
        self.host.array[:] = SENTINEL
        self.before = self.host.array.copy()
        self.perm = oracle.permutation(n)
        self.dst_addrs = np.uint64(self.host.ptr) + self.perm.astype(np.uint64) * np.uint64(self.stride)

    def check(self):
        want = oracle.expected_scatter(self.before, self.tokens, self.perm, self.t, self.stride)
        n_bad = int(np.count_nonzero(self.host.array != want))
        assert n_bad == 0, "%d mismatched bytes" % n_bad


SCATTER_CASES = [(8192, 4096), (2048, 65536), (2048, 512), (256, 4096), (97, 1000), (3, 48), (1, 16), (5, 12),
                 (4096, 2048)]


@pytest.mark.parametrize("n,t", SCATTER_CASES)
def test_zero_copy_scatter_tokens_parity(n, t):
    log("zero_copy_scatter n=%d t=%d" % (n, t))
    c = Offload(n, t)
    table = gfd_amd.DeviceBuffer(n * 8)
    table.upload(c.dst_addrs)
    gfd_amd.zero_copy_scatter_tokens(table.ptr, c.src.ptr, t, n)
    gfd_amd.synchronize()
    c.check()


# Few tokens are cut into pieces as in the gather, for the offload grid's 16
# waves: 4 x 64 KiB -> 16 of 16 KiB, 2 x 1 MiB -> 16 of 128 KiB, 5 x 24 KiB ->
# 10 of 12 KiB; with a 16-byte floor 3 x 4 KiB -> 12 of 1 KiB and 6 x 8200 B
# stays whole.
@pytest.mark.parametrize("n,t,min_piece", [(4, 65536, 4096), (2, 1 << 20, 4096), (5, 24576, 4096), (3, 4096, 16),
                                           (6, 8200, 16)])
def test_zero_copy_scatter_tokens_split_into_pieces(n, t, min_piece, monkeypatch):
    log("zero_copy_scatter pieces n=%d t=%d min_piece=%d" % (n, t, min_piece))
    monkeypatch.setenv("GFD_ZC_MIN_PIECE", str(min_piece))
    c = Offload(n, t)
    table = gfd_amd.DeviceBuffer(n * 8)
    table.upload(c.dst_addrs)
    for lds in ("0", "1"):
        monkeypatch.setenv("GFD_ZC_LDS", lds)
        c.host.array[:] = SENTINEL
        gfd_amd.zero_copy_scatter_tokens(table.ptr, c.src.ptr, t, n)
        gfd_amd.synchronize()
        c.check()


@pytest.mark.parametrize("waves,unroll", [(16, 4), (64, 16), (256, 8), (4, 4)])
def test_zero_copy_scatter_launch_shapes(waves, unroll, monkeypatch):
    """Bytes do not depend on the launch shape (GFD_ZCS_WAVES / _UNROLL)."""
    log("zero_copy_scatter shape waves=%d U=%d" % (waves, unroll))
    monkeypatch.setenv("GFD_ZCS_WAVES", str(waves))
    monkeypatch.setenv("GFD_ZCS_UNROLL", str(unroll))
    c = Offload(1000, 1040, seed=waves)
    table = gfd_amd.DeviceBuffer(c.n * 8)
    table.upload(c.dst_addrs)
    gfd_amd.zero_copy_scatter_tokens(table.ptr, c.src.ptr, c.t, c.n)
    gfd_amd.synchronize()
    c.check()


def test_zero_copy_scatter_host_table_and_coherent_destination():
    """The destination table may itself live in pinned host memory, and the
    destination may be fine-grained (coherent) host memory."""
    log("zero_copy_scatter host table, coherent dst")
    c = Offload(512, 4096, flags=gfd_amd.HOST_COHERENT)
    table = gfd_amd.HostBuffer(c.n * 8)
    table.array.view(np.uint64)[:] = c.dst_addrs
    gfd_amd.zero_copy_scatter_tokens(table.ptr, c.src.ptr, c.t, c.n)
    gfd_amd.synchronize()
    c.check()


def test_zero_copy_scatter_zero_count_is_noop_and_bad_args_rejected():
    gfd_amd.zero_copy_scatter_tokens(None, None, 4096, 0)
    with pytest.raises(gfd_amd.GfdError):
        gfd_amd.zero_copy_scatter_tokens(None, None, 4096, 4)
    src = gfd_amd.DeviceBuffer(4096)
    table = gfd_amd.DeviceBuffer(8)
    with pytest.raises(gfd_amd.GfdError):
        gfd_amd.zero_copy_scatter_tokens(table.ptr, src.ptr, 0, 1)
    with pytest.raises(gfd_amd.GfdError):
        gfd_amd.zero_copy_scatter_tokens(table.ptr, src.ptr, 4096, -1)


@pytest.mark.parametrize("n,t", [(8192, 4096), (2048, 65536)])
def test_gather_offload_round_trip(n, t):
    """Full-size round trip: gather the scattered tokens into HBM, clear the
    host region, offload them back in the same order: the host region must
    come back byte for byte, gaps included."""
    log("gather -> offload round trip n=%d t=%d" % (n, t))
    stride = 2 * t
    host = gfd_amd.HostBuffer(n * stride)
    oracle.fill_tokens(host.array, n, t, stride)
    original = host.array.copy()
    perm = oracle.permutation(n)
    addrs = np.uint64(host.ptr) + perm.astype(np.uint64) * np.uint64(stride)
    table = gfd_amd.DeviceBuffer(n * 8)
    table.upload(addrs)
    dev = gfd_amd.DeviceBuffer(n * t)
    gfd_amd.zero_copy_gather_tokens(table.ptr, dev.ptr, t, n)
    gfd_amd.synchronize()
    host.array.reshape(n, 2, t)[:, 0, :] = 0  # tokens gone, gaps (0xEE) kept
    gfd_amd.zero_copy_scatter_tokens(table.ptr, dev.ptr, t, n)
    gfd_amd.synchronize()
    n_bad = int(np.count_nonzero(host.array != original))
    assert n_bad == 0, "%d bytes differ after the round trip" % n_bad


@pytest.mark.parametrize("table_in", ["device", "host"])
def test_zero_copy_sg_offload_ragged(table_in):
    """The generic SG kernel moves HBM -> host lists too: ragged sizes,
    misaligned addresses, disjoint host destinations with gaps."""
    log("zero_copy SG offload ragged, table in %s" % table_in)
    rng = np.random.default_rng(9)
    sizes = rng.integers(1, 9000, 700)
    src = gfd_amd.DeviceBuffer(int(sizes.sum()) + 64 * len(sizes))
    data = rng.integers(0, 256, src.nbytes, dtype=np.uint8)
    src.upload(data)
    host = gfd_amd.HostBuffer(int(sizes.sum()) + 40 * len(sizes) + 4096)
    host.array[:] = SENTINEL
    want = host.array.copy()
    entries = (gfd_amd.SGEntry * len(sizes))()
    a = np.frombuffer(entries, dtype=np.uint64).reshape(len(sizes), 3)
    s_off, d_off = 3, 0
    for i, sz in enumerate(sizes):
        sz = int(sz)
        d_off += int(rng.integers(0, 40))
        a[i] = (host.ptr + d_off, src.ptr + s_off, sz)
        want[d_off:d_off + sz] = data[s_off:s_off + sz]
        d_off += sz
        s_off += sz + int(rng.integers(0, 64))
    raw = np.frombuffer(entries, dtype=np.uint8)
    if table_in == "device":
        tbl = gfd_amd.DeviceBuffer(raw.nbytes)
        tbl.upload(raw)
    else:
        tbl = gfd_amd.HostBuffer(raw.nbytes)
        tbl.array[:] = raw
    gfd_amd.zero_copy_gather(tbl.ptr, len(sizes))
    gfd_amd.synchronize()
    n_bad = int(np.count_nonzero(host.array != want))
    assert n_bad == 0, "%d mismatched bytes" % n_bad
