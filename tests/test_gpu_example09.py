"""The known-answer workload of examples/09_sg_warp_spec.cu on SGWarpSpecSession.

Data (09:334-340): TOTAL_TOKENS = 1024 tokens of TOKEN_DIM = 1024 fp32
values, token t, value d = sin((t*31 + d) * 0.01), in pinned host memory.
Routing token t -> expert t % 8 (09:370-388), one list per expert with
list_id = expert, one workgroup with one compute wave (09:359-361).

- Host pre-fill (09:352-432): every landed byte is compared with the source
  (the example allows 1e-5 per float; a copy is exact, so bytes are compared),
  and the MoE consumer's per-entry L2 norm, stored at out[list_id * count + i]
  (09:44-65), is compared with an fp64 reference: relative tolerance 1e-5
  (fp32 sum of 1024 squares of values <= 1 in magnitude).  The example itself
  only checks that each norm is finite (09:424-431).
- Linear compat (09:444-497): one list of 256 entries mapping token i to slot
  i (sg_compat::linear_to_sg_entries), bytes compared.
- GPU submission (09:503-575): the expert lists are submitted by the
  workgroup's submitter wave from a device entry table grouped by expert;
  bytes compared and per-list u32-word checksums exact."""
import sys

import numpy as np
import pytest

import gfd_amd
import oracle

pytestmark = pytest.mark.gpu

TOTAL_TOKENS, TOKEN_DIM, NUM_EXPERTS = 1024, 1024, 8
TOKEN_SIZE = TOKEN_DIM * 4
PER_EXPERT = TOTAL_TOKENS // NUM_EXPERTS
NORM_RTOL = 1e-5


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert gfd_amd.device_count() > 0, "no GPU visible to libgfd_amd.so"
    assert gfd_amd.lib().gfd_set_device(0) == 0


@pytest.fixture(scope="module")
def data():
    host = gfd_amd.HostBuffer(TOTAL_TOKENS * TOKEN_SIZE)
    t = np.arange(TOTAL_TOKENS, dtype=np.int64)[:, None]
    d = np.arange(TOKEN_DIM, dtype=np.int64)[None, :]
    vals = np.sin((t * 31 + d).astype(np.float32) * np.float32(0.01)).astype(np.float32)
    host.array[:] = vals.reshape(-1).view(np.uint8)
    dst = gfd_amd.DeviceBuffer(TOTAL_TOKENS * TOKEN_SIZE)
    return host, dst, vals


def expert_order():
    """Token ids in list order: expert e's list holds e, e + 8, e + 16, ..."""
    return np.concatenate([np.arange(e, TOTAL_TOKENS, NUM_EXPERTS) for e in range(NUM_EXPERTS)])


def entries_for(host, dst, tokens):
    tokens = np.asarray(tokens, dtype=np.uint64)
    return gfd_amd.device_sg_entries(np.uint64(host.ptr) + tokens * np.uint64(TOKEN_SIZE),
                                     np.uint64(dst.ptr) + tokens * np.uint64(TOKEN_SIZE), TOKEN_SIZE,
                                     tag=(tokens % np.uint64(NUM_EXPERTS)).astype(np.uint32))


def test_example09_host_prefill_l2norm(data):
    host, dst, vals = data
    log("example 09: host pre-fill, %d expert lists, L2-norm consumer" % NUM_EXPERTS)
    dst.fill(0)
    out = gfd_amd.DeviceBuffer(TOTAL_TOKENS * 4)
    out.fill(0)
    order = expert_order()
    ent = entries_for(host, dst, order)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=1, idle_limit_ms=5000)
    try:
        for e in range(NUM_EXPERTS):
            sess.submit_sg_list(ent[e * PER_EXPERT:(e + 1) * PER_EXPERT], e)
        sess.launch_l2norm(out.ptr, TOTAL_TOKENS)
        sess.synchronize()
        st = sess.stats()
    finally:
        sess.close()
    assert (dst.download() == host.array).all(), "landed bytes differ from the source"
    got = out.download().view(np.float32)
    assert np.isfinite(got).all()
    # out[list_id * count + i] is the norm of token order[list_id * count + i]
    want = np.sqrt((vals.astype(np.float64) ** 2).sum(axis=1))[order]
    np.testing.assert_allclose(got.astype(np.float64), want, rtol=NORM_RTOL, atol=0)
    assert st["units_done"] == TOTAL_TOKENS and st["lists_done"] == NUM_EXPERTS


def test_example09_linear_compat(data):
    host, dst, _ = data
    log("example 09: linear compat, one list of 256 entries")
    dst.fill(0)
    batch = 256
    ent = entries_for(host, dst, np.arange(batch))
    ent["tag"] = 0
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=1, idle_limit_ms=5000)
    try:
        sess.submit_sg_list(ent, 0)
        sess.launch()
        sess.synchronize()
    finally:
        sess.close()
    got = dst.download()
    assert (got[:batch * TOKEN_SIZE] == host.array[:batch * TOKEN_SIZE]).all()
    assert (got[batch * TOKEN_SIZE:] == 0).all(), "bytes past the list were written"


def test_example09_gpu_submitted_expert_lists(data):
    host, dst, _ = data
    log("example 09: GPU-submitted expert lists")
    dst.fill(0)
    order = expert_order()
    ent = entries_for(host, dst, order)
    d_ent = gfd_amd.DeviceBuffer(ent.nbytes)
    d_ent.upload(ent.view(np.uint8))
    sums = gfd_amd.DeviceBuffer(gfd_amd.MAX_SG_LISTS * 8)
    sums.fill(0)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=1, idle_limit_ms=5000)
    try:
        sess.launch_gpu_submit(d_ent.ptr, PER_EXPERT, NUM_EXPERTS, sums.ptr)
        sess.synchronize(extra_gpu_lists=NUM_EXPERTS)
    finally:
        sess.close()
    assert (dst.download() == host.array).all()
    got = sums.download().view(np.uint64)
    for e in range(NUM_EXPERTS):
        toks = order[e * PER_EXPERT:(e + 1) * PER_EXPERT]
        want = sum(oracle.u32_word_checksum(host.array[int(t) * TOKEN_SIZE:(int(t) + 1) * TOKEN_SIZE])
                   for t in toks) & oracle.MASK64
        assert int(got[e]) == want, "expert %d checksum" % e
