"""The reference's include surface compiles for reference-style callers.

tests/cxx/direct_transfer.cpp is a host program written like the
reference's examples/02_direct_transfer.cu (#include <gfd/gfd.h>,
StagingPool, CpuPollingThread, init_copy_engine / init_direct_ce / start,
submit_direct); it is compiled with g++ and linked against libgfd_amd.so.
tests/cxx/sessions_e2e.hip is device code written like the reference's
test/test_sg_e2e.cu and test/test_db_small_tiles.cu (<gfd/sg_warp_spec.cuh>,
<gfd/warp_spec.cuh>, GFD_SG_WARP_SPEC_KERNEL, GFD_WARP_SPEC_KERNEL_DB, the
sessions' launch templates); it is compiled with hipcc for gfx950.
tests/cxx/sg_gpu_submit.hip follows test/test_sg_gpu_submit.cu: a
caller-written transfer / compute / submitter kernel launched with
hipLaunchKernelGGL and bracketed by session.get_poller()->start() / stop().
All are built into a temporary directory here; the GPU test runs the copies that
build() leaves in tests/cxx/_build.  Also: every reference header name
exists and <gfd/gfd.h> compiles on its own in plain C++17."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")

# Header names of the reference's include/gfd/ (include/gfd/*.h, *.cuh).
REFERENCE_HEADERS = [
    "copy_engine.h", "cpu_polling.h", "descriptor_queue.h", "device.cuh", "device_primitives.cuh", "gfd.h",
    "log.h", "pcie_topology.h", "sg_device_primitives.cuh", "sg_task_queue.h", "sg_warp_spec.cuh",
    "staging_pool.h", "tiled_queue.h", "warp_spec.cuh", "warp_spec_session.h",
]


def test_every_reference_header_name_exists():
    missing = [h for h in REFERENCE_HEADERS if not os.path.isfile(os.path.join(INC, "gfd", h))]
    assert not missing, missing


def test_umbrella_header_compiles_alone_in_plain_cxx(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    src = tmp_path / "t.cpp"
    src.write_text(
        "#include <gfd/gfd.h>\n"
        "int main() {\n"
        "  gfd::TopologyConfig t = gfd::discover_topology(1);\n"
        "  int b = 0, n = 0, s = 0; t.get_exclusive_cores(0, b, n, s);\n"
        "  gfd::StagingPool& p = gfd::StagingPool::instance(); (void)p;\n"
        "  gfd::WarpSpecConfig c; c.total_tokens = 1024; c.token_size = 4096;\n"
        "  return (int)c.effective_tokens_per_chunk() + t.recommended_ce_channels(1) + "
        "(int)sizeof(gfd::SGEntry) + (int)sizeof(gfd::Descriptor);\n"
        "}\n")
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", "-I" + INC, str(src)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr


def test_reference_style_callers_build(tmp_path):
    lib = os.path.join(ROOT, "gfd_amd", "libgfd_amd.so")
    if not os.path.isfile(lib):
        pytest.skip("libgfd_amd.so not built")
    if shutil.which("g++") is None or shutil.which("hipcc") is None:
        pytest.skip("g++ or hipcc not available")
    r = subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "tests", "cxx"), "OUT=%s" % tmp_path],
                       capture_output=True, text=True, timeout=600)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and "recognized feature" not in l)
    assert r.returncode == 0, err
    for name in ("direct_transfer", "sessions_e2e", "sg_gpu_submit"):
        assert os.path.isfile(tmp_path / name), name
    # The host program resolves the library's C++ API from libgfd_amd.so.
    nm = subprocess.run(["nm", "-D", "--undefined-only", str(tmp_path / "direct_transfer")], capture_output=True,
                        text=True, timeout=60).stdout
    for sym in ("CpuPollingThread", "submit_direct", "StagingPool", "discover_topology"):
        assert sym in nm, sym


def test_exclusive_core_partition_on_synthetic_topologies(tmp_path):
    """TopologyConfig::get_exclusive_cores on hand-built multi-GPU, multi-NUMA
    topologies (tests/cxx/topology_partition.cpp): the reference's values on
    consecutively numbered nodes (its include/gfd/pcie_topology.h:41-60),
    disjoint equal shares of each node's own cores on every layout, and the
    edge cases.  Host code only: it runs without a GPU."""
    lib = os.path.join(ROOT, "gfd_amd", "libgfd_amd.so")
    if not os.path.isfile(lib):
        pytest.skip("libgfd_amd.so not built")
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "topology_partition"
    r = subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "tests", "cxx"), "OUT=%s" % tmp_path, str(exe)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    # Built outside tests/cxx/_build, so the program's relative rpath does not
    # reach gfd_amd/: name the library's folder instead.
    env = dict(os.environ)
    env["LD_LIBRARY_PATH"] = os.pathsep.join(p for p in (os.path.dirname(lib), env.get("LD_LIBRARY_PATH")) if p)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60, env=env)
    assert r.returncode == 0, r.stderr
    assert "PASSED" in r.stdout


def test_sg_counter_layout_and_helpers(tmp_path):
    """The SG session's device-counter layout and the helpers device code uses
    to reach it without reading the host queue (tests/cxx/queue_layouts.cpp):
    counters right after d_list_done[MAX_SG_LISTS], sg_list_done_words() back
    to that array, sg_idle_ticks() in 100 MHz ticks with 0 meaning 30 s.
    Header-only host code."""
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "queue_layouts"
    r = subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "tests", "cxx"), "OUT=%s" % tmp_path, str(exe)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "PASSED" in r.stdout
