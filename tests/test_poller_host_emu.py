"""The product poller stack on the CPU: gfd_amd/csrc/{cpu_polling,copy_engine,
sdma,gather_engine,staging_pool,direct_submit}.cpp built unchanged with g++
(AddressSanitizer + UBSan) against an emulated HSA runtime and HIP shim
(tests/host_emu).  Emulated copy engines run their copies in order per engine
and evaluate a dependency by polling the dependency signal's value when the
copy reaches the head of its engine, as the SDMA engines do.

Host threads follow the kernels' device protocols:
- SG mode (reference src/batch_processor.cpp:307-446, include/gfd/
  sg_warp_spec.cuh:95-262): lists tagged list_id << 32 | i, FLAG_LAST_IN_TILE
  on the last entry, a wait on d_list_done[list_id], then a checksum of what
  landed.  The four cases of the GPU test of the kernel-driven mode
  (including lists split over several batches) and the page-scattered lists
  of the CPU-producer GPU test.  The product library switches this mode off;
  the emulation build (GFD_HOST_EMULATION) keeps it so its logic stays tested.
- Queue mode (reference src/cpu_polling.cpp:337-490): contiguous and
  scattered destinations, then a wait on done_idx.
- SdmaQueue signal-slot reuse: a copy that depends on a slot's previous
  occupant must have polled it before the slot is handed on.
- StagingPool sets taken and released by Queue pollers, with the fallback to
  the poller's own staging.
- Registered host memory mapped at another GPU address is refused as a
  copy source.
Every landed byte is compared with the expected image, list checksums exactly.
"""
import fcntl
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EMU = os.path.join(HERE, "host_emu")
BIN = os.path.join(EMU, "_build", "poller_emu")


@pytest.fixture(scope="module")
def poller_emu():
    if shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include/hsa"):
        pytest.skip("g++ or the HSA headers are not available")
    # One build at a time: parallel test workers each reach this fixture.
    os.makedirs(os.path.join(EMU, "_build"), exist_ok=True)
    with open(os.path.join(EMU, "_build", ".lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        subprocess.check_call(["make", "-s", "-j8", "-C", EMU], timeout=600)
    return BIN


@pytest.fixture(scope="module")
def poller_emu_protect():
    if shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include/hsa"):
        pytest.skip("g++ or the HSA headers are not available")
    os.makedirs(os.path.join(EMU, "_build_protect"), exist_ok=True)
    with open(os.path.join(EMU, "_build_protect", ".lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        subprocess.check_call(["make", "-s", "-j8", "-C", EMU, "protect"], timeout=600)
    return os.path.join(EMU, "_build_protect", "poller_emu")


@pytest.fixture(scope="module")
def poller_emu_tsan():
    if shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include/hsa"):
        pytest.skip("g++ or the HSA headers are not available")
    os.makedirs(os.path.join(EMU, "_build_tsan"), exist_ok=True)
    with open(os.path.join(EMU, "_build_tsan", ".lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        subprocess.check_call(["make", "-s", "-j8", "-C", EMU, "tsan"], timeout=600)
    return os.path.join(EMU, "_build_tsan", "poller_emu")


def run(binary, args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    e.setdefault("GFD_EMU_STALL_MS", "3000")
    # Also catch writes through pointers into stack frames that have returned.
    e.setdefault("ASAN_OPTIONS", "detect_stack_use_after_return=1")
    p = subprocess.run([binary] + [str(a) for a in args], capture_output=True, text=True, timeout=120, env=e)
    out = p.stdout + p.stderr
    assert p.returncode == 0, "poller_emu %s exited %d:\n%s" % (" ".join(map(str, args)), p.returncode, out[-3000:])
    assert "pass" in p.stdout, out[-3000:]
    return out


def test_sdma_signal_slot_reuse_waits_for_pending_dependents(poller_emu):
    run(poller_emu, ["sdma_slot_reuse"])


@pytest.mark.parametrize("case", ["split_small_tokens", "ragged", "host_flags", "one_entry_lists", "pages"])
def test_sg_mode_lists(poller_emu, case):
    run(poller_emu, ["sg", case, 2, 1])


def test_sg_mode_split_lists_slow_engines(poller_emu):
    # Slower copies keep well over a thousand copies in flight across batches.
    run(poller_emu, ["sg", "split_small_tokens", 2, 7], env={"GFD_EMU_COPY_NS": "3000"})


@pytest.mark.parametrize("n,t,scattered", [(2048, 512, 0), (8192, 4096, 0), (4096, 1000, 1), (300, 1000, 1),
                                           (1, 4096, 0)])
def test_queue_mode(poller_emu, n, t, scattered):
    run(poller_emu, ["queue", n, t, scattered, 2, 3])


def zero_copy_launches(out):
    return [int(l.split(":")[1]) for l in out.splitlines() if l.startswith("zero-copy launches:")]


@pytest.mark.parametrize("path,nruns", [("direct", 1), ("direct", 8), ("direct", 40), ("queue", 1), ("queue", 8),
                                        ("queue", 100)])
def test_ragged_entries_over_destination_runs(poller_emu, path, nruns):
    # Entries of 1..8999 bytes at every alignment: staged gathers with one
    # copy per chunk or per run piece, and per-run copies.  A Direct list with
    # one destination run (about 3 MiB) takes the zero-copy route; with
    # several runs it does not.
    out = run(poller_emu, ["ragged", path, 700, nruns, 2, 3])
    if path == "direct":
        assert zero_copy_launches(out) == [1 if nruns == 1 else 0] * 2, out[-2000:]


@pytest.mark.parametrize("n,max_entry", [(5, 200000), (40, 70000), (63, 9000), (3, 100000)])
def test_direct_short_ragged_list_cut_into_pieces(poller_emu, n, max_entry):
    # A short destination-contiguous list of large ragged entries: the
    # zero-copy route cuts the entries into pieces of at least 4 KiB (16-byte
    # multiples) for the kernel's waves; every byte is compared, under
    # AddressSanitizer, against the list's own image.
    out = run(poller_emu, ["ragged", "direct", n, 1, 2, 5], env={"GFD_EMU_MAX_ENTRY": str(max_entry)})
    assert zero_copy_launches(out) == [1] * 2, out[-2000:]


@pytest.mark.parametrize("zc_min,launches", [(0, 1), (64 << 20, 0)])
def test_direct_zero_copy_minimum(poller_emu, zc_min, launches):
    # The one-run list of about 3 MiB: on the zero-copy route with no minimum,
    # staged once the minimum (GFD_DIRECT_ZC_MIN_BYTES) is above its size (the
    # staged route's zero-copy head is off here, so no kernel runs at all).
    out = run(poller_emu, ["ragged", "direct", 700, 1, 2, 3],
              env={"GFD_DIRECT_ZC_MIN_BYTES": str(zc_min), "GFD_DIRECT_ZC_HEAD_BYTES": "0"})
    assert zero_copy_launches(out) == [launches] * 2, out[-2000:]


@pytest.mark.parametrize("head,launches", [(512 << 10, 1), (0, 0)])
def test_direct_staged_route_with_zero_copy_head(poller_emu, head, launches):
    # The same contiguous ragged list above the zero-copy route's limit (set
    # to 1 MiB here): staged through the gather workers and the copy engines,
    # with its first 512 KiB moved by the zero-copy kernel meanwhile, or with
    # the head switched off.  Every byte is compared either way.
    out = run(poller_emu, ["ragged", "direct", 700, 1, 2, 3],
              env={"GFD_DIRECT_ZC_MAX_BYTES": str(1 << 20), "GFD_DIRECT_ZC_HEAD_BYTES": str(head)})
    assert zero_copy_launches(out) == [launches] * 2, out[-2000:]


@pytest.mark.parametrize("tiles,T,C,ts,whole,hbm", [(8, 128, 32, 4096, 0, 1), (8, 128, 32, 4096, 1, 1),
                                                    (16, 64, 64, 1000, 0, 1), (4, 256, 16, 2048, 0, 0),
                                                    (100, 32, 8, 512, 0, 1)])
def test_tiled_mode(poller_emu, tiles, T, C, ts, whole, hbm):
    # Tiled mode (reference src/batch_processor.cpp:69-298): per-tile
    # cumulative progress words after each chunk's copies, in HBM (8-byte
    # copies chained behind the data and the previous progress write) or in
    # host memory; the shapes of the GPU test of the kernel-driven mode.
    run(poller_emu, ["tiled", tiles, T, C, ts, whole, hbm, 2, 3])


def test_tiled_mode_whole_tiles_slow_engines(poller_emu):
    # Four batches of one tile in flight together on slow engines: each
    # progress write must land after the previous one.
    run(poller_emu, ["tiled", 8, 128, 32, 4096, 1, 1, 2, 5], env={"GFD_EMU_COPY_NS": "3000"})


def test_staging_pool_sets_and_fallback(poller_emu):
    # StagingPool (reference include/gfd/staging_pool.h:50-176): the set
    # selection rule (the requested NUMA node first, then any node), acquire /
    # release / a request larger than the buffers (-1), then four Queue
    # pollers: two take the pool's two sets, one whose region is larger than
    # the buffers and one that finds every set taken allocate their own
    # staging (src/cpu_polling.cpp:160-245).  Every poller's rounds are
    # checked byte for byte, and both sets are free once the pollers are gone.
    run(poller_emu, ["staging_pool", 2, 5])


def test_registered_host_memory_at_another_gpu_address_is_not_a_copy_source(poller_emu):
    # Host memory the runtime reports as locked (registered) with a GPU-side
    # address different from its host address cannot be handed to SDMA copies
    # or the zero-copy kernel by its host address; at the same address it can.
    run(poller_emu, ["locked_source"])


def test_direct_looks_up_pinned_sources_on_every_call(poller_emu):
    """A source range found pinned by one submit_direct call whose
    registration is gone by the next (freed, its addresses reused by pageable
    memory) must not reach the zero-copy kernel: the second call looks it up
    again and takes the staged route.  The emulated kernel aborts on a source
    that is not pinned, as the GPU would fault."""
    out = run(poller_emu, ["stale_pinned"])
    assert "call 0, zero-copy launches 1" in out and "call 1, zero-copy launches 0" in out, out[-2000:]


@pytest.mark.parametrize("workers", [0, 1, 3, 15])
def test_gather_engine_whole_and_pipelined_runs(poller_emu, workers):
    """GatherEngine alone: whole-list runs (the reference's static W+1 split,
    src/parallel_gather.cpp:90-116, each worker's slice handed over in its
    mailbox line), pipelined runs and parallel list scans in random order on
    one engine, over uniform, ragged and empty entries; every byte of every
    run is compared with the memcpy image, and again after the next run with
    the sources inverted in between, so a worker still copying after run()
    returned would show.  A 200 us spin limit makes some jobs meet sleeping
    workers."""
    out = run(poller_emu, ["gather_mix", workers, 300, workers + 5], env={"GFD_GATHER_SPIN_US": "200"})
    assert "gather mix: pass" in out, out[-2000:]


# The same stack built with ThreadSanitizer instead: the poller, gather
# workers, copy engines and the host threads that play the kernels' protocols
# must show no data race (a report makes the run exit 66).
@pytest.mark.parametrize("args", [["sg", "split_small_tokens", 2, 1], ["sg", "pages", 2, 1],
                                  ["queue", 4096, 1000, 1, 2, 3], ["ragged", "direct", 700, 1, 2, 3],
                                  ["tiled", 8, 128, 32, 4096, 1, 1, 2, 5], ["staging_pool", 2, 5],
                                  ["sdma_slot_reuse"], ["gather_mix", 7, 60, 16]])
def test_no_data_race_under_tsan(poller_emu_tsan, args):
    out = run(poller_emu_tsan, args, env={"TSAN_OPTIONS": "halt_on_error=0 exitcode=66", "GFD_GATHER_SPIN_US": "200"})
    assert "ThreadSanitizer" not in out, out[-3000:]


@pytest.mark.parametrize("case", ["split_small_tokens", "pages"])
def test_sg_mode_abort_workloads_under_stack_protector(poller_emu_protect, case):
    """The two SG-mode workloads that aborted on MI355X with "stack smashing
    detected" (5 lists of 1 KiB entries, three longer than the 1024-entry
    batch threshold; page-scattered 4 KiB entries, two lists longer than
    4096), at those shapes, with every function of the poller stack carrying
    a stack canary and glibc's checked copies (-fstack-protector-all
    -D_FORTIFY_SOURCE=3, -O3): no canary is overwritten and every byte lands."""
    run(poller_emu_protect, ["sg", case, 3, 1])


def test_direct_routes_through_the_zero_copy_worker(poller_emu):
    """submit_direct with the persistent zero-copy worker on (emulated: the
    records are copied on the calling thread, each side checked to be pinned
    or device memory): short, ragged, one-entry and contiguous lists with
    pinned sources become worker jobs; pageable sources and a list above the
    zero-copy limit take the other routes.  Every byte is compared."""
    out = run(poller_emu, ["worker_direct"])
    assert out.count(": worker") == 6 and out.count(": other route") == 2, out[-2000:]


@pytest.mark.parametrize("n,t,scattered,want_jobs", [(2048, 512, 0, True), (2048, 2048, 1, True),
                                                      (2048, 65536, 0, False)])
def test_queue_batches_through_the_zero_copy_worker(poller_emu, n, t, scattered, want_jobs):
    """Queue mode with the worker on: batches of at most 4 MiB (small tokens,
    contiguous or scattered destinations) become worker jobs, larger ones are
    staged for the copy engines as before; done_idx and every byte checked."""
    out = run(poller_emu, ["queue", n, t, scattered, 2, 1], env={"GFD_ZC_WORKER": "1"})
    jobs = int(out.split("zero-copy worker jobs: ")[1].split()[0])
    assert (jobs > 0) == want_jobs, out[-2000:]
