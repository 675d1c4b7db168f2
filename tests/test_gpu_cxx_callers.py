"""Reference-style C++ callers, run on the GPU (built by build() into
tests/cxx/_build; see tests/test_cxx_callers.py for what they are).

direct_transfer: the known-answer check of the reference's
examples/02_direct_transfer.cu (token i filled with i & 0xFF, every byte
compared) through submit_direct, in order and in a seeded random order, with
the poller's Queue staging taken from the StagingPool.
sessions_e2e: the reference's test/test_sg_e2e.cu (floats i + 1 landed by an
SGWarpSpecSession, every one compared) and test/test_db_small_tiles.cu
(double-buffered tiles, per-token sums (t + 1) * dim at 1-7 tiles), with the
session poller's stats printed as examples/07_warp_spec_simple.cu:283 does.
sg_gpu_submit: the reference's test/test_sg_gpu_submit.cu flow: a
caller-launched transfer / compute / submitter kernel bracketed by
session.get_poller()->start() and stop(), floats i + 1 checked, twice on one
session, then a launch through the session."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "tests", "cxx", "_build")


@pytest.mark.parametrize("prog", ["direct_transfer", "sessions_e2e", "sg_gpu_submit"])
def test_reference_style_program(prog):
    path = os.path.join(BUILD, prog)
    assert os.path.isfile(path), "%s is not built: run __graft_entry__.build()" % path
    print("running %s" % prog, flush=True)
    sys.stdout.flush()
    r = subprocess.run([path], capture_output=True, text=True, timeout=100)
    out = r.stdout + r.stderr
    print(out[-2000:], flush=True)
    assert r.returncode == 0, out[-3000:]
    assert "PASSED" in r.stdout, out[-3000:]
