"""gfd_moe_route_noalloc (the allocation-free variant of gfd_moe_route, for
callers that cannot allocate) against gfd_moe_route: the same per-expert
offsets and row lists, bit for bit, on two calls in a row, the second with
fewer tokens (the scratch keeps the first call's pairs), plus the oracle;
and a clear error beyond the scratch maximum, with nothing launched."""
import sys

import numpy as np
import pytest

import gfd_amd
import oracle

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_moe_route_noalloc_matches_moe_route():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0
    L = gfd_amd.lib()
    for T, E in ((4096, 64), (1000, 16)):
        log("moe_route_noalloc T=%d E=%d" % (T, E))
        logits = oracle.moe_logits(T, E)
        want_off, want_rows = oracle.moe_lists(oracle.moe_top2(logits), E)
        d_logits = gfd_amd.DeviceBuffer(logits.nbytes)
        d_logits.upload(logits)
        d_top2, d_off, d_rows = (gfd_amd.DeviceBuffer(2 * T * 4), gfd_amd.DeviceBuffer((E + 1) * 4),
                                 gfd_amd.DeviceBuffer(2 * T * 4))
        n_off, n_rows = gfd_amd.DeviceBuffer((E + 1) * 4 + 64), gfd_amd.DeviceBuffer(2 * T * 4 + 64)
        n_off.fill(0xA5)
        n_rows.fill(0xA5)
        assert L.gfd_moe_route(d_logits.ptr, T, E, d_top2.ptr, d_off.ptr, d_rows.ptr, None) == 0
        assert L.gfd_moe_route_noalloc(d_logits.ptr, T, E, n_off.ptr, n_rows.ptr, None) == 0, L.gfd_last_error()
        gfd_amd.synchronize()
        ref_off, ref_rows = d_off.download().view(np.int32), d_rows.download().view(np.int32)
        got_off = n_off.download()
        got_rows = n_rows.download()
        assert (got_off[:(E + 1) * 4].view(np.int32) == ref_off).all()
        assert (got_rows[:2 * T * 4].view(np.int32) == ref_rows).all()
        assert (got_off[(E + 1) * 4:] == 0xA5).all() and (got_rows[2 * T * 4:] == 0xA5).all()
        assert (ref_off == want_off).all() and (ref_rows == want_rows).all()


def test_moe_route_noalloc_rejects_more_tokens_than_the_scratch_holds():
    assert gfd_amd.lib().gfd_set_device(0) == 0
    L = gfd_amd.lib()
    dummy = gfd_amd.DeviceBuffer(4096)
    rc = L.gfd_moe_route_noalloc(dummy.ptr, 65537, 64, dummy.ptr, dummy.ptr, None)
    assert rc != 0
    assert b"65536" in L.gfd_last_error()
