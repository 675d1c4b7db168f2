"""GPU parity of the MoE-routed gather through SGWarpSpecSession (the SG MoE
workload of the reference's examples/09_sg_warp_spec.cu:78-294 run through
the session API, include/gfd/sg_warp_spec.cuh): routing on the GPU, per-expert
row lists built by GPU submitter waves and posted with the sg:: primitives,
rows copied by the session's transfer waves, a bf16 RMSNorm on every landed
list by the compute wave, or by up to three compute waves sharing each list.  Rows byte-exact against the oracle, RMSNorm within
one bf16 ulp of the fp32 oracle, list / entry / byte counts exact."""
import numpy as np
import pytest

import gfd_amd
import oracle
from test_gpu_moe import Moe

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


def expected_lists(offsets, rows_per_list):
    counts = np.diff(offsets.astype(np.int64))
    return int(np.sum((counts + rows_per_list - 1) // rows_per_list))


def run_session(m, sess, with_norm, rows_per_list, eps=1e-6):
    m.d_dst.fill(0xCD)
    m.d_out.fill(0xCD)
    n = 2 * m.T
    sess.reset()
    sess.launch_moe(m.host.ptr, m.stride, m.T, m.d_offsets.ptr, m.d_rows.ptr, m.E, n, m.row_bytes, m.d_dst.ptr,
                    m.d_out.ptr if with_norm else None, m.d_weight.ptr, eps, rows_per_list)
    gfd_amd.synchronize()  # the kernel ends once every list has landed
    sess.synchronize(0)
    return sess.stats()


# cw: compute waves sharing each landed list (the RMSNorm consumer splits a
# list's rows between them); 1 = the reference's single compute wave.
@pytest.mark.parametrize("T,E,dim,rpl,blocks,cw", [(4096, 64, 7168, 8, 0, 1), (4096, 64, 7168, 64, 16, 1),
                                                   (4096, 64, 7168, 2, 0, 1), (64, 8, 512, 4, 2, 1),
                                                   (300, 5, 1024, 7, 0, 1), (1000, 16, 2048, 1, 8, 1),
                                                   (4096, 64, 7168, 32, 0, 3), (4096, 64, 7168, 7, 4, 2),
                                                   (300, 5, 1024, 1, 2, 3), (4096, 64, 7168, 48, 40, 3)])
def test_moe_through_session(T, E, dim, rpl, blocks, cw):
    print("moe session T=%d E=%d dim=%d rows/list=%d blocks=%d compute waves=%d" % (T, E, dim, rpl, blocks, cw),
          flush=True)
    m = Moe(T, E, dim)
    m.route()
    assert (m.d_rows.download().view(np.int32) == m.row_token).all()
    n = 2 * T
    rows = m.expected_rows()
    ref = oracle.rmsnorm_rows(oracle.bf16_to_f32(rows), oracle.bf16_to_f32(m.weight), 1e-6)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=cw, num_blocks=blocks, idle_limit_ms=10000)
    try:
        for with_norm in (False, True, True):  # two overlapped launches: the session's state carries over
            st = run_session(m, sess, with_norm, rpl)
            assert st["error_bits"] == 0
            assert st["lists_done"] == expected_lists(m.offsets, rpl)
            assert st["units_done"] == n and st["bytes"] == n * m.row_bytes
            got = m.d_dst.download()
            assert (got[:n * m.row_bytes].view(np.uint16).reshape(n, dim) == rows).all()
            assert (got[n * m.row_bytes:] == 0xCD).all()
            out = m.d_out.download()
            if not with_norm:
                assert (out == 0xCD).all()
                continue
            y = oracle.bf16_to_f32(out[:n * m.row_bytes].view(np.uint16).reshape(n, dim))
            assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6)
            assert np.mean(oracle.f32_to_bf16(ref) == oracle.f32_to_bf16(y)) > 0.99
            assert (out[n * m.row_bytes:] == 0xCD).all()
    finally:
        sess.close()


def test_moe_session_with_host_lists_queued_before_launch():
    """Host lists queued before launch_moe land in the same launch, and the
    session's lists_done counts them: the GPU submitter must wait for those
    and its own lists before it raises stop, or transfer waves holding later
    GPU lists would leave them uncopied.  Two host lists of 32 tokens each go
    ahead of a launch whose rows must all land byte-exact, with the host
    lists' tokens and every count exact."""
    T, E, dim, rpl = 1000, 16, 2048, 4
    m = Moe(T, E, dim)
    m.route()
    n = 2 * T
    rows = m.expected_rows()
    total = expected_lists(m.offsets, rpl)
    k, t = 32, 4096
    side_host = gfd_amd.HostBuffer(2 * k * t)
    side_host.array[:] = np.random.default_rng(9).integers(0, 256, 2 * k * t, dtype=np.uint8)
    side_dst = gfd_amd.DeviceBuffer(2 * k * t)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=8, idle_limit_ms=10000)
    try:
        for launch in range(2):
            print("moe session with 2 host lists queued, launch %d" % launch, flush=True)
            sess.reset()
            m.d_dst.fill(0xCD)
            side_dst.fill(0)
            for l in range(2):
                idx = np.arange(l * k, (l + 1) * k, dtype=np.uint64)
                ent = np.zeros(k, dtype=gfd_amd.DEVICE_SG_ENTRY_DTYPE)
                ent["src"] = side_host.ptr + idx * t
                ent["dst"] = side_dst.ptr + idx * t
                ent["size"] = t
                sess.submit_sg_list(ent, 1000 + l)
            sess.launch_moe(m.host.ptr, m.stride, m.T, m.d_offsets.ptr, m.d_rows.ptr, m.E, n, m.row_bytes,
                            m.d_dst.ptr, None, m.d_weight.ptr, 1e-6, rpl)
            gfd_amd.synchronize()
            sess.synchronize(0)
            st = sess.stats()
            assert st["error_bits"] == 0
            assert st["lists_done"] == total + 2
            assert st["units_done"] == n + 2 * k and st["bytes"] == n * m.row_bytes + 2 * k * t
            got = m.d_dst.download()
            assert (got[:n * m.row_bytes].view(np.uint16).reshape(n, dim) == rows).all()
            assert (side_dst.download() == side_host.array).all()
    finally:
        sess.close()


def test_moe_session_trace():
    """The per-list device timeline: every list of the launch is recorded once,
    in ring order, with claimed <= ready <= landed; each workgroup's record
    brackets its lists and the workgroups' list counts add up; the session's
    results are unchanged; with tracing off there is nothing to read."""
    T, E, dim, rpl = 4096, 64, 7168, 48
    m = Moe(T, E, dim)
    m.route()
    n = 2 * T
    rows = m.expected_rows()
    total = expected_lists(m.offsets, rpl)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=3, num_blocks=32, idle_limit_ms=10000)
    try:
        sess.enable_trace(1024)
        for launch in range(2):  # records are cleared for every launch
            print("traced moe session launch %d" % launch, flush=True)
            st = run_session(m, sess, True, rpl)
            assert st["error_bits"] == 0 and st["lists_done"] == total
            got = m.d_dst.download()[:n * m.row_bytes].view(np.uint16).reshape(n, dim)
            assert (got == rows).all()
            lists, blocks = sess.trace()
            assert len(lists) == 1024 and len(blocks) == 32
            used, rest = lists[:total], lists[total:]
            assert (rest["claimed"] == 0).all() and (rest["landed"] == 0).all()
            assert sorted(used["list_id"].tolist()) == list(range(total))
            assert (used["claimed"] > 0).all()
            assert (used["claimed"] <= used["ready"]).all() and (used["ready"] <= used["landed"]).all()
            assert (used["block"] < 32).all()
            assert int(blocks["lists"].sum()) == total
            # Where each workgroup ran (XCC_ID << 32 | HW_ID): MI355X has 8 XCCs,
            # and 32 workgroups are spread over more than one.
            xcc = (blocks["hw"] >> np.uint64(32)) & np.uint64(0xF)
            assert (xcc < 8).all() and len(set(xcc.tolist())) > 1, blocks["hw"]
            for b in range(32):
                mine = used[used["block"] == b]
                assert len(mine) == int(blocks["lists"][b])
                assert blocks["start"][b] > 0 and blocks["exit"][b] >= blocks["start"][b]
                if len(mine):
                    assert blocks["start"][b] <= mine["claimed"].min()
                    assert blocks["exit"][b] >= mine["landed"].max()
            span_us = (used["landed"].max() - blocks["start"].min()) / gfd_amd.SG_TRACE_TICKS_PER_US
            print("first start to last landing: %.1f us" % span_us, flush=True)
            assert 0 < span_us < 10e6
        sess.enable_trace(0)
        run_session(m, sess, False, rpl)
        with pytest.raises(gfd_amd.GfdError):
            sess.trace()
    finally:
        sess.close()


@pytest.mark.parametrize("with_norm,cw", [(False, 1), (True, 1), (True, 3)])
def test_moe_session_skips_out_of_range_rows(with_norm, cw):
    """A routing entry outside the token range is reported (error bit 16) and
    its row skipped (an empty entry, which the staged-row RMSNorm never
    sees); every other row lands, and with the RMSNorm every other row is
    normalised."""
    print("moe session with one out-of-range row, norm=%s compute waves=%d" % (with_norm, cw), flush=True)
    m = Moe(64, 8, 1024)
    m.route()
    rt = m.row_token.copy()
    rt[5] = m.T + 3
    m.d_rows.upload(rt)
    n = 2 * m.T
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=cw, num_blocks=2, idle_limit_ms=10000)
    try:
        m.d_dst.fill(0xCD)
        m.d_out.fill(0xCD)
        sess.reset()
        sess.launch_moe(m.host.ptr, m.stride, m.T, m.d_offsets.ptr, m.d_rows.ptr, m.E, n, m.row_bytes, m.d_dst.ptr,
                        m.d_out.ptr if with_norm else None, m.d_weight.ptr, 1e-6, 16)
        gfd_amd.synchronize()
        with pytest.raises(gfd_amd.GfdError):
            sess.synchronize(0)
        assert sess.stats()["error_bits"] & 16
        got = m.d_dst.download()[:n * m.row_bytes].view(np.uint16).reshape(n, m.dim)
        rows = m.values[np.clip(rt, 0, m.T - 1)]
        keep = np.arange(n) != 5
        assert (got[keep] == rows[keep]).all()
        assert (got[5].view(np.uint8) == 0xCD).all()
        out = m.d_out.download()
        if not with_norm:
            assert (out == 0xCD).all()
            return
        y = out[:n * m.row_bytes].view(np.uint16).reshape(n, m.dim)
        assert (y[5].view(np.uint8) == 0xCD).all()
        ref = oracle.rmsnorm_rows(oracle.bf16_to_f32(rows[keep]), oracle.bf16_to_f32(m.weight), 1e-6)
        yk = oracle.bf16_to_f32(y[keep])
        assert np.all(np.abs(yk - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6)
    finally:
        sess.close()


@pytest.mark.parametrize("staged", ["1", "0"])
def test_moe_session_rmsnorm_staged_and_list_mode(staged, monkeypatch):
    """The RMSNorm consumer both ways: rows staged in LDS by the transfer wave
    (the default) and per landed list read back from HBM
    (GFD_SG_STAGED_ROWS=0), at the full 14 KiB rows and 3 compute waves;
    rows byte-exact, RMSNorm within bf16 of the fp32 oracle."""
    print("moe session RMSNorm, GFD_SG_STAGED_ROWS=%s" % staged, flush=True)
    monkeypatch.setenv("GFD_SG_STAGED_ROWS", staged)
    m = Moe(4096, 64, 7168)
    m.route()
    n = 2 * m.T
    rows = m.expected_rows()
    ref = oracle.rmsnorm_rows(oracle.bf16_to_f32(rows), oracle.bf16_to_f32(m.weight), 1e-6)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=3, num_blocks=40, idle_limit_ms=10000)
    try:
        st = run_session(m, sess, True, 48)
        assert st["error_bits"] == 0 and st["units_done"] == n
        got = m.d_dst.download()
        assert (got[:n * m.row_bytes].view(np.uint16).reshape(n, m.dim) == rows).all()
        y = oracle.bf16_to_f32(m.d_out.download()[:n * m.row_bytes].view(np.uint16).reshape(n, m.dim))
        assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6)
    finally:
        sess.close()


def test_moe_session_rejects_bad_arguments():
    m = Moe(64, 8, 512)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=2, idle_limit_ms=1000)
    try:
        with pytest.raises(gfd_amd.GfdError):  # 65 rows per list
            sess.launch_moe(m.host.ptr, m.stride, m.T, m.d_offsets.ptr, m.d_rows.ptr, m.E, 2 * m.T, m.row_bytes,
                            m.d_dst.ptr, None, None, 1e-6, 65)
        with pytest.raises(gfd_amd.GfdError):  # more rows than the entry pool holds
            sess.launch_moe(m.host.ptr, m.stride, m.T, m.d_offsets.ptr, m.d_rows.ptr, m.E, 16385, m.row_bytes,
                            m.d_dst.ptr, None, None, 1e-6, 16)
        with pytest.raises(gfd_amd.GfdError):  # RMSNorm needs whole 1 KiB row blocks
            sess.launch_moe(m.host.ptr, m.stride, m.T, m.d_offsets.ptr, m.d_rows.ptr, m.E, 2 * m.T, 1000,
                            m.d_dst.ptr, m.d_out.ptr, m.d_weight.ptr, 1e-6, 16)
    finally:
        sess.close()
