"""CPU checks of bench.py's measurement helpers and its command-line contract:
the parser behind roofline.traffic (rocprofv3 counter files), the summary of
an SG session's per-list timeline, and the refusal of more than one GPU."""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
import gfd_amd  # noqa: E402

HEADER = ('"Correlation_Id","Dispatch_Id","Agent_Id","Queue_Id","Process_Id","Thread_Id","Grid_Size","Kernel_Id",'
          '"Kernel_Name","Workgroup_Size","LDS_Block_Size","Scratch_Size","VGPR_Count","Accum_VGPR_Count",'
          '"SGPR_Count","Counter_Name","Counter_Value","Start_Timestamp","End_Timestamp"')


def row(dispatch, grid, name, counter, value):
    return '%d,%d,"Agent 1",1,1,1,%d,1,"%s",256,0,0,8,0,48,"%s",%f,0,1' % (dispatch, dispatch, grid, name, counter,
                                                                            value)


def test_pmc_parser_keeps_the_calibration_launches_and_the_full_size_gathers(tmp_path):
    rows = [row(1, 65536, "__amd_rocclr_fillBufferAligned", "FETCH_SIZE", 16.0)]
    # Five calibration copies first, then a later copy that must not count.
    rows += [row(2 + i, 131072, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 16390.0 + i) for i in range(5)]
    # Five contiguous calibration gathers on the full grid, before anything else launches the kernel.
    rows += [row(7 + i, 16384, "void (anonymous namespace)::zc_gather_tokens<false>(...)", "FETCH_SIZE",
                 16440.0 + i) for i in range(5)]
    # The set-up launch on 16 bytes (one workgroup), then 12 launches of the job.
    rows.append(row(12, 256, "void (anonymous namespace)::zc_gather_tokens<false>(...)", "FETCH_SIZE", 1.0))
    rows += [row(13 + i, 16384, "void (anonymous namespace)::zc_gather_tokens<false>(...)", "FETCH_SIZE",
                 16457.0 + i) for i in range(12)]
    rows.append(row(25, 131072, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 99999.0))
    # Another counter's rows are ignored.
    rows.append(row(26, 16384, "void (anonymous namespace)::zc_gather_tokens<false>(...)", "WRITE_SIZE", 5.0))
    p = tmp_path / "p_counter_collection.csv"
    p.write_text("\n".join([HEADER] + rows) + "\n")
    copies, contig, gathers = bench.parse_pmc_counters(str(p), "FETCH_SIZE")
    assert copies == [16390.0 + i for i in range(5)]
    assert contig == [16440.0 + i for i in range(5)]
    assert gathers == [16457.0 + i for i in range(12)]
    copies, contig, gathers = bench.parse_pmc_counters(str(p), "WRITE_SIZE")
    assert copies == [] and contig == [5.0] and gathers == []


def test_session_timeline_summary():
    ticks = gfd_amd.SG_TRACE_TICKS_PER_US
    lists = np.zeros(4, dtype=gfd_amd.SG_TRACE_LIST_DTYPE)
    # (claimed, ready, landed) in us after t0 = 1000 ticks; blocks 0 and 1.
    for k, (c, r, l, b) in enumerate([(1, 3, 50, 0), (2, 5, 60, 1), (50, 52, 90, 0), (60, 61, 70, 1)]):
        lists[k] = (1000 + c * ticks, 1000 + r * ticks, 1000 + l * ticks, b, k)
    blocks = np.zeros(2, dtype=gfd_amd.SG_TRACE_BLOCK_DTYPE)
    blocks[0] = (1000, 1000 + 95 * ticks, 2, 0)
    blocks[1] = (1000 + 1 * ticks, 1000 + 80 * ticks, 2, 0)
    s = bench.session_timeline(lists, blocks, 4)
    assert s["first_copy_us"] == 3.0
    assert s["last_landing_us"] == 90.0
    assert s["last_exit_us"] == 95.0
    assert s["workgroup_last_landing_us"] == [70.0, 80.0, 90.0]
    assert s["claim_to_ready_mean_us"] == round((2 + 3 + 2 + 1) / 4, 2)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""
