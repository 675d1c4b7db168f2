"""Scattered H2D gather benchmark on one MI355X.

Workload (one "step"): gather 8192 tokens x 4 KiB (32 MiB) scattered at 2x
stride in pinned host memory, in a seeded random order, into one contiguous
HBM buffer.  Also measured in the same run: 2048 x 64 KiB (KV-cache pages),
2048 x {512 B, 1 KiB, 2 KiB}, the contiguous-copy link peak, per-token
hipMemcpyAsync, the CPU ParallelGather restatement on the host cores, and the
reverse path (offload of the same layouts from HBM to pinned host).  The
zero-copy kernel's HBM-side traffic comes from two rocprofv3 --pmc passes run
as child processes at the end (about 30 s).
Timing: W warm-up + K timed iterations, P50 (examples/04_benchmark.cu:58-90).
GB/s = bytes / (us * 1e3).

    python bench.py [--gpus 1] [--steps 50] [--warmup 15] [--only zc|direct|...]

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import ctypes
import csv
import glob
import json
import os
import shutil
import signal
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import gfd_amd  # noqa: E402

PCIE_GEN5_X16_GBPS = 32.0 * 16 * 128.0 / 130.0 / 8.0  # 63.0 GB/s per direction

# Bytes one zc_gather_tokens launch moves at 8192 x 4 KiB, from two
# rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of `bench.py --only zc,calib`,
# each scaled by the same counter on a 32 MiB device-to-device copy
# (FETCH x 1.99853, WRITE x 1.0).  Reads are host-link reads through the L2's
# external interface; writes land in HBM.  A default run measures them again
# (measure_traffic); these profiled values stand in only if that fails.
ZC_TRAFFIC_8192x4KB = {"read_bytes": 32891 * 1024, "write_bytes": 32772 * 1024}
METRIC = "scattered H2D GB/s + % of PCIe5 x16 peak at 8192x4KB and 2048x64KB"
DIRECT_ZC_MAX = 8 << 20  # submit_direct's default zero-copy route limit (bytes)
DIRECT_ZC_MIN = 64 << 10  # lists up to this size take the staged route


def direct_route(nbytes):
    """The route submit_direct takes by default for a destination-contiguous
    list of scattered tokens with pinned sources."""
    if nbytes <= DIRECT_ZC_MIN:
        return "staged SDMA"
    return "zero-copy kernel" if nbytes <= DIRECT_ZC_MAX else "staged SDMA + zero-copy head"
DIRECT_ZC_HEAD = 2 << 20  # and the zero-copy head of larger staged lists
# MoE through SGWarpSpecSession: workgroups, compute waves sharing each list
# in the RMSNorm, rows per GPU-built list (swept: 24-128 workgroups, 1-3
# compute waves, 2-64 rows per list).
MOE_SESSION_BLOCKS, MOE_SESSION_COMPUTE_WAVES, MOE_SESSION_ROWS_PER_LIST = 40, 3, 48
MOE_SESSION_HELPERS = -1  # transfer helper waves per workgroup (negative: the session's default rule)
PD = ctypes.POINTER(ctypes.c_double)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def p50(x):
    return float(np.percentile(np.asarray(x, dtype=np.float64), 50))


def gbps(nbytes, us):
    return nbytes / (us * 1e3) if us > 0 else 0.0


class Layout:
    """n tokens of t bytes at 2t stride in pinned host memory, seeded order."""

    def __init__(self, oracle, n, t, flags=gfd_amd.HOST_DEFAULT):
        self.n, self.t, self.stride = n, t, 2 * t
        self.bytes = n * t
        self.host = gfd_amd.HostBuffer(n * self.stride, flags)
        oracle.fill_tokens(self.host.array, n, t, self.stride)
        self.perm = oracle.permutation(n)
        self.expected = oracle.expected_gather(self.host.array, self.perm, t, self.stride)
        self.src_addrs = np.uint64(self.host.ptr) + self.perm.astype(np.uint64) * np.uint64(self.stride)
        self.dst = gfd_amd.DeviceBuffer(self.bytes)
        self.table = gfd_amd.DeviceBuffer(n * 8)
        self.table.upload(self.src_addrs)
        self.entries = gfd_amd.make_entries(self.src_addrs, self.dst.ptr, t)
        tok = np.zeros((n, 2), np.uint64)
        tok[:, 0] = self.src_addrs
        tok[:, 1] = np.arange(n, dtype=np.uint64)
        self.tokens = gfd_amd.DeviceBuffer(tok.nbytes)
        self.tokens.upload(tok)

    def verify(self, what):
        self.dst_ok = bool((self.dst.download() == self.expected).all())
        if not self.dst_ok:
            raise SystemExit("PARITY FAILURE: %s (%d x %d)" % (what, self.n, self.t))
        self.dst.fill(0)
        return True


def host_info():
    import platform

    info = {"logical_cpus": os.cpu_count(), "allowed_cpus": len(os.sched_getaffinity(0))}
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["cpu_model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        info["numa_nodes"] = open("/sys/devices/system/node/online").read().strip()
    except OSError:
        pass
    info["machine"] = platform.machine()
    # SMT: hardware threads per physical core among the CPUs this process may use.
    cores = set()
    allowed = sorted(os.sched_getaffinity(0))
    for c in allowed:
        try:
            base = "/sys/devices/system/cpu/cpu%d/topology/" % c
            cores.add((open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip()))
        except OSError:
            cores = set()
            break
    if cores:
        info["physical_cores"] = len(cores)
        info["threads_per_core"] = round(len(allowed) / len(cores), 2)
        info["smt"] = len(allowed) > len(cores)
    return info


CPU_COLD_REGIONS = 8  # source regions the cold CPU baseline rotates over (8 x 64 MiB)


def cpu_baseline(oracle, seconds, info):
    """The reference CPU ParallelGather restated (oracle/oracle.c), timed on
    this host's cores: 8192 x 4 KiB into a pinned staging buffer.

    value: cold source.  The gather rotates over CPU_COLD_REGIONS source
    regions of 64 MiB (512 MiB in all, more than the host's last-level
    cache), each with the same token layout, so every gather reads tokens no
    recent gather has touched, as a KV cache in host DRAM would be.
    warm_value: the same gather repeated on one region (its tokens stay in
    the CPU caches between iterations)."""
    allowed = sorted(os.sched_getaffinity(0))
    workers = max(0, min(15, len(allowed) - 1))
    cpus = allowed[:workers + 1]
    n, t = 8192, 4096
    perm = oracle.permutation(n)
    srcs = []
    for _ in range(CPU_COLD_REGIONS):
        b = gfd_amd.HostBuffer(n * 2 * t)
        oracle.fill_tokens(b.array, n, t, 2 * t)
        srcs.append(b)
    staging = gfd_amd.HostBuffer(n * t)
    entries = [oracle.make_entries(b.ptr, 0, perm, t, 2 * t) for b in srcs]
    expect = lambda k: oracle.expected_gather(srcs[k].array, perm, t, 2 * t)
    # The restated gather and the product's gather engine take turns in
    # blocks over the whole window, so that both see the same load on the
    # host's memory (other tenants of a shared host move it by 10-30%).
    blocks = max(1, int(round(seconds / 2.0)))
    cold, warm, prod = [], [], []
    t_start = time.time()
    t_log = t_start + 2.5
    k = 0
    for blk in range(blocks):
        pool = oracle.GatherPool(workers, cpus)
        try:
            if blk == 0:
                pool.gather(entries[0], n, staging.array, 0)
                if not (staging.array == expect(0)).all():
                    raise SystemExit("PARITY FAILURE: CPU baseline")
            t_end = t_start + seconds * (blk + 1) / blocks - 0.25
            while time.time() < t_end:
                for _ in range(20):
                    cold.extend(pool.time(entries[k % CPU_COLD_REGIONS], n, staging.array, 0, 1).tolist())
                    k += 1
                if time.time() < t_start + 0.25 * seconds or len(warm) < 200:
                    warm.extend(pool.time(entries[0], n, staging.array, 0, 20).tolist())
                if time.time() > t_log:
                    log("  cpu baseline: %d cold gathers (P50 %.1f us), %d warm (P50 %.1f us), product %d (P50 %s us)" % (
                        len(cold), p50(cold), len(warm), p50(warm), len(prod),
                        ("%.1f" % p50(prod)) if prod else "-"))
                    t_log += 2.5
            if blk == blocks - 1:
                pool.gather(entries[CPU_COLD_REGIONS - 1], n, staging.array, 0)
                if not (staging.array == expect(CPU_COLD_REGIONS - 1)).all():
                    raise SystemExit("PARITY FAILURE: CPU baseline (last region)")
        finally:
            pool.close()
            os.sched_setaffinity(0, allowed)
        prod.extend(product_gather([b.ptr for b in srcs], perm, n, t, staging, cpus, workers, expect,
                                   iters=max(100, 3000 // blocks))["times_us"])
    us, us_warm = p50(cold), p50(warm)
    product = {"us_p50": round(p50(prod), 2), "GBps": round(gbps(n * t, p50(prod)), 3), "workers": workers,
               "cpus": list(cpus[:workers + 1]), "gathers": len(prod), "regions": CPU_COLD_REGIONS,
               "blocks": blocks}
    out = {
        "value": round(gbps(n * t, us), 3), "unit": "GB/s", "cores": workers + 1, "kind": "port",
        "sample": "8192 x 4KiB ParallelGather into pinned staging, cold source: rotating over %d regions of "
                  "64 MiB, %d gathers (%.0f s), P50 %.1f us; W=%d workers + caller on CPUs %s, AVX-512=%s" % (
                      CPU_COLD_REGIONS, len(cold), seconds, us, workers, cpus, oracle.has_avx512()),
        "warm_value": round(gbps(n * t, us_warm), 3),
        "warm_sample": "the same gather repeated on one 64 MiB region (source in CPU caches): %d gathers, "
                       "P50 %.1f us" % (len(warm), us_warm),
    }
    out["product_gather"] = product
    # Flat copies of the figures the record keeps (it drops nested objects).
    out["restated_gather_us"] = round(us, 2)
    out["product_gather_us"] = product["us_p50"]
    out["product_gather_GBps"] = product["GBps"]
    for k in ("physical_cores", "threads_per_core", "smt"):
        if k in info:
            out[k] = info[k]
    for b in srcs:
        b.free()
    # The CPU-only layout: 256 x 4 KiB from a 2 MiB source into 1 MiB of
    # staging, with W = 15 workers (the reference's setting; it oversubscribes
    # a host with fewer than 16 CPUs) and with W = 7.
    c1 = {}
    n1 = 256
    src1 = gfd_amd.HostBuffer(n1 * 2 * t)
    oracle.fill_tokens(src1.array, n1, t, 2 * t)
    perm1 = oracle.permutation(n1)
    stg1 = gfd_amd.HostBuffer(n1 * t)
    ent1 = oracle.make_entries(src1.ptr, 0, perm1, t, 2 * t)
    expect1 = oracle.expected_gather(src1.array, perm1, t, 2 * t)
    for w in (15, 7):
        wcpus = [allowed[i % len(allowed)] for i in range(w + 1)]  # threads share CPUs when W+1 > CPUs
        pool = oracle.GatherPool(w, wcpus)
        try:
            pool.gather(ent1, n1, stg1.array, 0)
            if not (stg1.array == expect1).all():
                raise SystemExit("PARITY FAILURE: CPU baseline 256 x 4KiB")
            tt = []
            t_end = time.time() + 1.5
            while time.time() < t_end:
                tt.extend(pool.time(ent1, n1, stg1.array, 0, 200).tolist())
        finally:
            pool.close()
            os.sched_setaffinity(0, allowed)
        c1["W%d" % w] = {"us_p50": round(p50(tt), 2), "GBps": round(gbps(n1 * t, p50(tt)), 3),
                         "threads": w + 1, "cpus": len(set(wcpus)),
                         "oversubscribed": w + 1 > len(allowed), "iterations": len(tt)}
        # The product's gather engine on the same list and threads.
        pg = product_gather([src1.ptr], perm1, n1, t, stg1, wcpus, w, lambda k: expect1, iters=2000)
        c1["W%d" % w]["product_gather"] = {"us_p50": pg["us_p50"], "GBps": pg["GBps"]}
    out["c1_256x4KB"] = c1
    for w in (15, 7):
        out["c1_256x4KB_W%d_us" % w] = c1["W%d" % w]["us_p50"]
        out["c1_256x4KB_W%d_product_us" % w] = c1["W%d" % w]["product_gather"]["us_p50"]
    log("  cpu baseline 256 x 4KiB: %s" % c1)
    return out


def product_gather(region_ptrs, perm, n, t, staging, cpus, workers, expected, iters=3000):
    """The product's gather engine (gfd_bench_host_gather: the Direct path's
    staging step without the copies) on the layout of cpu_baseline: tokens at
    2x stride in each region, the same order, W workers pinned to cpus[1..]
    and the caller on cpus[0]; gather k reads region k % len(region_ptrs)."""
    lists = [gfd_amd.make_entries(np.uint64(r) + perm.astype(np.uint64) * np.uint64(2 * t), 0, t)
             for r in region_ptrs]
    ptrs = (ctypes.c_void_p * len(lists))(*[ctypes.cast(l, ctypes.c_void_p) for l in lists])
    cpu_ids = (ctypes.c_int * (workers + 1))(*cpus[:workers + 1])
    tt = np.zeros(iters)
    rc = gfd_amd.lib().gfd_bench_host_gather(ptrs, len(lists), n, staging.ptr, 2 << 20, workers, cpu_ids,
                                             len(lists) * 2, iters, tt.ctypes.data_as(PD))
    assert rc == 0, gfd_amd.lib().gfd_last_error()
    # The last gather read region (warmup + iters - 1) % len(regions).
    last = (len(lists) * 2 + iters - 1) % len(lists)
    if not (staging.array == expected(last)).all():
        raise SystemExit("PARITY FAILURE: product host gather (region %d)" % last)
    return {"us_p50": round(p50(tt), 2), "GBps": round(gbps(n * t, p50(tt)), 3), "workers": workers,
            "cpus": list(cpus[:workers + 1]), "gathers": iters, "regions": len(lists), "times_us": tt.tolist()}


def bench_peak(nbytes, iters, warmup):
    src = gfd_amd.HostBuffer(nbytes)
    src.array[:] = 1
    dst = gfd_amd.DeviceBuffer(nbytes)
    out = {}
    for ns in (1, 4):
        t = np.zeros(iters)
        rc = gfd_amd.lib().gfd_bench_memcpy_contiguous(dst.ptr, src.ptr, nbytes, ns, warmup, iters,
                                                       t.ctypes.data_as(PD))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        out["hip_%d_stream" % ns] = round(gbps(nbytes, p50(t)), 3)
    mask = ctypes.c_uint32(0)
    for ch, pin in ((1, 1), (2, 1), (4, 1), (2, 0)):
        t = np.zeros(iters)
        rc = gfd_amd.lib().gfd_bench_sdma_contiguous(dst.ptr, src.ptr, nbytes, ch, pin, warmup, iters,
                                                     t.ctypes.data_as(PD), ctypes.byref(mask))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        out["sdma_%dch_%s" % (ch, "pinned" if pin else "auto")] = round(gbps(nbytes, p50(t)), 3)
    out["sdma_engine_mask"] = "0x%x" % mask.value
    return out


def run_zero_copy(L, iters, warmup):
    """Zero-copy tokens kernel.  us_p50: launch call until the host sees the
    grid's completion word (the library's own wait); wall_sync_us_p50: launch
    until hipStreamSynchronize returns; kernel_*: HIP events on the stream."""
    wall = np.zeros(iters)
    ev = np.zeros(iters)
    rc = gfd_amd.lib().gfd_bench_zero_copy_tokens(L.table.ptr, L.dst.ptr, L.t, L.n, warmup, iters,
                                                  wall.ctypes.data_as(PD), ev.ctypes.data_as(PD))
    assert rc == 0, gfd_amd.lib().gfd_last_error()
    L.verify("zero-copy")
    sig = np.zeros(iters)
    rc = gfd_amd.lib().gfd_bench_zero_copy_tokens_signal(L.table.ptr, L.dst.ptr, L.t, L.n, warmup, iters,
                                                         sig.ctypes.data_as(PD))
    assert rc == 0, gfd_amd.lib().gfd_last_error()
    L.verify("zero-copy (signalled)")
    return {"us_p50": round(p50(sig), 2), "GBps": round(gbps(L.bytes, p50(sig)), 3),
            "wall_sync_us_p50": round(p50(wall), 2),
            "kernel_us_mean": round(float(ev.mean()), 2), "kernel_us_p50": round(p50(ev), 2),
            "kernel_GBps": round(gbps(L.bytes, float(ev.mean())), 3),
            "wall_over_kernel": round(p50(sig) / float(ev.mean()), 4)}


def run_direct(poller, L, iters, warmup):
    """submit_direct as configured: lists up to 8 MiB on the zero-copy route,
    larger ones staged for the copy engines with their first 2 MiB moved by
    the zero-copy kernel meanwhile.  Also the staged SDMA route alone
    (staged_sdma: no kernel at all)."""
    t = np.zeros(iters)

    def timed_calls(what):
        rc = gfd_amd.lib().gfd_bench_submit_direct(poller._h, ctypes.cast(L.entries, ctypes.c_void_p), L.n, warmup,
                                                   iters, t.ctypes.data_as(PD))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        L.verify(what)
        return {"us_p50": round(p50(t), 2), "GBps": round(gbps(L.bytes, p50(t)), 3)}

    out = timed_calls("direct")
    head = poller.set_direct_zero_copy_head_bytes(DIRECT_ZC_HEAD)
    out["route"] = direct_route(L.bytes) + (" of %d KiB" % (head >> 10) if L.bytes > DIRECT_ZC_MAX else "")
    poller.set_direct_zero_copy_max_bytes(0)  # also switches the head off
    out["staged_sdma"] = timed_calls("direct (staged SDMA)")
    poller.set_direct_zero_copy_max_bytes(DIRECT_ZC_MAX)
    return out


def _busy_union(iv):
    """Total length of the union of [start, end) intervals."""
    tot, cur_s, cur_e = 0, None, None
    for a, b in sorted(iv):
        if cur_e is None or a > cur_e:
            if cur_e is not None:
                tot += cur_e - cur_s
            cur_s, cur_e = a, b
        else:
            cur_e = max(cur_e, b)
    if cur_e is not None:
        tot += cur_e - cur_s
    return tot


def sdma_occupancy(copies, t0, t1):
    """SDMA engine activity inside the window [t0, t1] (ns, HSA system clock):
    fraction of the window with any engine busy, each engine's busy fraction,
    the host-link rate while busy, the wait before the first copy starts and
    the tail after the last copy ends."""
    c = copies[(copies["start_ns"] >= t0) & (copies["end_ns"] <= t1)]
    win = max(1, t1 - t0)
    if len(c) == 0:
        return None
    iv = [(int(a), int(b)) for a, b in zip(c["start_ns"], c["end_ns"])]
    busy = _busy_union(iv)
    per_engine = {}
    for e in np.unique(c["engine"]):
        m = c["engine"] == e
        per_engine["0x%x" % int(e)] = round(_busy_union([(int(a), int(b)) for a, b in
                                                         zip(c["start_ns"][m], c["end_ns"][m])]) / win, 4)
    return {"copies": int(len(c)), "bytes": int(c["bytes"].sum()), "window_us": round(win / 1e3, 2),
            "busy_frac_any": round(busy / win, 4),
            "busy_frac_per_engine": per_engine, "link_GBps_while_busy": round(int(c["bytes"].sum()) / busy, 3),
            "first_copy_start_us": round((int(c["start_ns"].min()) - t0) / 1e3, 2),
            "tail_after_last_copy_us": round((t1 - int(c["end_ns"].max())) / 1e3, 2)}


def direct_timeline(poller, L, calls=20):
    """SDMA timeline of `calls` submit_direct calls (after the timed loop):
    median of each per-call figure of sdma_occupancy()."""
    poller.set_copy_timing(True)
    windows = []
    for _ in range(calls):
        t0 = poller.copy_clock_ns()
        us = poller.submit_direct(L.entries, L.n)
        t1 = poller.copy_clock_ns()
        assert us > 0
        windows.append((t0, t1))
    copies = poller.read_copy_times()
    poller.set_copy_timing(False)
    L.verify("direct (timed copies)")
    per = [o for o in (sdma_occupancy(copies[copies["path"] == 1], a, b) for a, b in windows) if o]
    if not per:
        return None
    med = lambda k: round(float(np.median([o[k] for o in per])), 4)
    engines = sorted(set(k for o in per for k in o["busy_frac_per_engine"]))
    return {"calls": len(per), "copies_per_call": med("copies"), "sdma_bytes_per_call": med("bytes"),
            "window_us": med("window_us"),
            "busy_frac_any": med("busy_frac_any"), "link_GBps_while_busy": med("link_GBps_while_busy"),
            "first_copy_start_us": med("first_copy_start_us"), "tail_after_last_copy_us": med("tail_after_last_copy_us"),
            "busy_frac_per_engine": {e: round(float(np.median([o["busy_frac_per_engine"].get(e, 0.0) for o in per])), 4)
                                     for e in engines}}


# The reference's published Direct points (README.md:60-65 and 86-89; in-order
# tokens at 2x stride, RTX PRO 5000, P50 of 50): tokens -> microseconds.
REFERENCE_DIRECT_4KB_US = {16: 9.7, 64: 14.2, 256: 31.0, 1024: 91.7, 2048: 170.2, 4096: 328.3, 8192: 645.0}
REFERENCE_DIRECT_64KB_US = {16: 41.4, 64: 96.7, 256: 360.8, 1024: 1269.0, 2048: 2534.8}


def run_short_lists(oracle, poller, iters, warmup):
    """Short lists of large entries, which the zero-copy kernels spread over
    their 64 waves: submit_direct on 4 tokens of 64 KiB (cut into pieces in
    the token kernel) and on 4 ragged entries of about 256 KiB (cut on the
    host), and gfd_zero_copy_gather on one 1 MiB entry with its table in HBM
    (sliced in the kernel; HIP events on a stream).  Each output is checked
    byte for byte."""
    out = {}
    L = Layout(oracle, 4, 65536)
    t = np.zeros(iters)
    rc = gfd_amd.lib().gfd_bench_submit_direct(poller._h, ctypes.cast(L.entries, ctypes.c_void_p), L.n, warmup,
                                               iters, t.ctypes.data_as(PD))
    assert rc == 0, gfd_amd.lib().gfd_last_error()
    L.verify("direct 4 x 64 KiB")
    out["direct_4x64KB"] = {"us_p50": round(p50(t), 2), "GBps": round(gbps(L.bytes, p50(t)), 3)}
    del L
    rng = np.random.default_rng(3)
    lib = gfd_amd.lib()
    for key, sizes in (("direct_ragged_4x256KB", [262144, 262160, 262128, 262144]),
                       ("zero_copy_sg_1x1MB", [1 << 20])):
        sizes = np.array(sizes, np.uint64)
        n, slot = len(sizes), int(sizes.max()) + 16
        host = gfd_amd.HostBuffer(slot * n)
        host.array[:] = rng.integers(0, 256, host.nbytes, dtype=np.uint8)
        order = rng.permutation(n).astype(np.uint64)
        dst = gfd_amd.DeviceBuffer(int(sizes.sum()))
        dst_offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.uint64)
        ent = np.zeros((n, 3), np.uint64)
        ent[:, 0] = np.uint64(dst.ptr) + dst_offs
        ent[:, 1] = np.uint64(host.ptr) + order * np.uint64(slot)
        ent[:, 2] = sizes
        if key.startswith("direct"):
            entries = (gfd_amd.SGEntry * n)()
            np.frombuffer(entries, dtype=np.uint64).reshape(n, 3)[:] = ent
            rc = lib.gfd_bench_submit_direct(poller._h, ctypes.cast(entries, ctypes.c_void_p), n, warmup, iters,
                                             t.ctypes.data_as(PD))
            assert rc == 0, lib.gfd_last_error()
            us = p50(t)
        else:
            tab = gfd_amd.DeviceBuffer(ent.nbytes)
            tab.upload(ent.view(np.uint8).reshape(-1))
            st, ea, eb = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
            lib.gfd_stream_create(ctypes.byref(st))
            lib.gfd_event_create(ctypes.byref(ea))
            lib.gfd_event_create(ctypes.byref(eb))
            ts = []
            for i in range(-warmup, iters):
                lib.gfd_event_record(ea, st)
                assert lib.gfd_zero_copy_gather(tab.ptr, n, st) == 0, lib.gfd_last_error()
                lib.gfd_event_record(eb, st)
                lib.gfd_event_synchronize(eb)
                ms = ctypes.c_float(0)
                lib.gfd_event_elapsed_ms(ctypes.byref(ms), ea, eb)
                if i >= 0:
                    ts.append(ms.value * 1000.0)
            lib.gfd_event_destroy(ea)
            lib.gfd_event_destroy(eb)
            lib.gfd_stream_destroy(st)
            us = p50(np.array(ts))
        got = dst.download()
        for i in range(n):
            so, do, s = int(order[i]) * slot, int(dst_offs[i]), int(sizes[i])
            if not (got[do:do + s] == host.array[so:so + s]).all():
                raise SystemExit("PARITY FAILURE: %s entry %d" % (key, i))
        out[key] = {"us_p50": round(us, 2), "GBps": round(gbps(int(sizes.sum()), us), 3), "entries": n}
    log("  short lists: %s" % {k: v["us_p50"] for k, v in out.items()})
    return out


def run_direct_sizes(oracle, poller, iters, warmup):
    """submit_direct over the token counts the reference publishes (4 KiB
    tokens: 16 ... 4096; 64 KiB tokens: 16 ... 1024), on the bench's layout
    (seeded random order, 2x stride), each checked byte-exact; the
    reference's figure beside each."""
    out = {}
    for t, ref in ((4096, REFERENCE_DIRECT_4KB_US), (65536, REFERENCE_DIRECT_64KB_US)):
        row = {}
        for n in sorted(ref):
            if (t == 4096 and n == 8192) or (t == 65536 and n == 2048):
                continue  # the main configurations, measured above
            L = Layout(oracle, n, t)
            tt = np.zeros(iters)
            rc = gfd_amd.lib().gfd_bench_submit_direct(poller._h, ctypes.cast(L.entries, ctypes.c_void_p), n, warmup,
                                                       iters, tt.ctypes.data_as(PD))
            assert rc == 0, gfd_amd.lib().gfd_last_error()
            L.verify("direct %d x %d" % (n, t))
            row[str(n)] = {"us_p50": round(p50(tt), 2), "GBps": round(gbps(n * t, p50(tt)), 3),
                           "route": direct_route(n * t),
                           "reference_us": ref[n], "reference_GBps": round(gbps(n * t, ref[n]), 2)}
            del L
        out["%dKB" % (t // 1024)] = row
        log("  direct sizes %d KiB: %s" % (t // 1024, {k: v["us_p50"] for k, v in row.items()}))
    return out


def run_worker_direct(oracle, iters, warmup):
    """submit_direct through the persistent zero-copy worker (a poller with
    set_zero_copy_worker on): the reference's published short lists (4 KiB
    tokens, 16 ... 1024; 64 KiB tokens, 16), few large tokens, and the
    config-4 sizes; each output checked byte for byte."""
    p = gfd_amd.CpuPollingThread(None, None, None, 16 << 20, numa_node=-1)
    out = {}
    try:
        assert p.init_direct_ce(), "init_direct_ce failed"
        p.set_zero_copy_worker(True)
        shapes = [(n, 4096) for n in (16, 64, 256, 1024)] + [(4, 65536), (16, 65536), (2048, 512), (2048, 1024),
                                                              (2048, 2048)]
        for n, t in shapes:
            L = Layout(oracle, n, t)
            tt = np.zeros(iters)
            jobs0 = p.zero_copy_worker_stats()["jobs"]
            rc = gfd_amd.lib().gfd_bench_submit_direct(p._h, ctypes.cast(L.entries, ctypes.c_void_p), n, warmup, iters,
                                                       tt.ctypes.data_as(PD))
            assert rc == 0, gfd_amd.lib().gfd_last_error()
            L.verify("direct through the worker %d x %d" % (n, t))
            assert p.zero_copy_worker_stats()["jobs"] == jobs0 + warmup + iters, "not through the worker"
            key = "%dx%s" % (n, ("%dKB" % (t // 1024)) if t >= 1024 else "%dB" % t)
            out[key] = {"us_p50": round(p50(tt), 2), "GBps": round(gbps(n * t, p50(tt)), 3)}
            ref = (REFERENCE_DIRECT_4KB_US if t == 4096 else REFERENCE_DIRECT_64KB_US if t == 65536 else {}).get(n)
            if ref:
                out[key]["reference_us"] = ref
            log("  direct through the worker %s: %s" % (key, out[key]))
            del L
        out["worker"] = p.zero_copy_worker_stats()
    finally:
        p.close()
    out["device_timeline"] = worker_device_timeline(oracle, iters)
    return out


def worker_device_timeline(oracle, calls):
    """The worker's own per-job timeline (GFD_ZC_WORKER_TRACE=1, a poller of
    its own; untimed): median us, after the last workgroup found the job, at
    which the last one held its records, the last one had copied its share
    and the last progress word was stored."""
    os.environ["GFD_ZC_WORKER_TRACE"] = "1"
    p = gfd_amd.CpuPollingThread(None, None, None, 16 << 20, numa_node=-1)
    out = {}
    try:
        assert p.init_direct_ce(), "init_direct_ce failed"
        p.set_zero_copy_worker(True)
        for n, t in ((16, 4096), (64, 4096), (2048, 512), (2048, 2048)):
            L = Layout(oracle, n, t)
            for _ in range(max(calls, 40)):
                assert p.submit_direct(L.entries, L.n) > 0
            L.verify("direct through the traced worker %d x %d" % (n, t))
            tl = p.zero_copy_worker_timeline(40).astype(np.int64)
            rel = (tl[:, :6] - tl[:, :1]) / 100.0  # 100 MHz ticks -> us
            m = np.median(rel, axis=0)
            out["%dx%d" % (n, t)] = {"records_us": round(float(m[1]), 2), "copied_us": round(float(m[3]), 2),
                                     "progress_us": round(float(m[5]), 2), "jobs": int(len(tl))}
            log("  worker device timeline %dx%d: %s" % (n, t, out["%dx%d" % (n, t)]))
            del L
    finally:
        p.close()
        os.environ.pop("GFD_ZC_WORKER_TRACE", None)
    return out


def run_direct_scattered(oracle, poller, iters, warmup):
    """GFD Direct with non-contiguous destinations, 8192 x 4 KiB tokens
    (scattered sources as in the main layout): 'pages' = a paged KV cache,
    token j lands in page slot s_j of 16384 (seeded permutation), so every
    token is its own destination run; 'blocks' = 40 contiguous destination
    blocks with 12 KiB gaps.  Output checked byte-exact with sentinel gaps."""
    n, t = 8192, 4096
    out = {}
    for name in ("pages", "blocks"):
        if name == "pages":
            offs = np.random.default_rng(0x5EED).permutation(2 * n)[:n].astype(np.uint64) * np.uint64(t)
            region = 2 * n * t
        else:
            per = -(-n // 40)
            offs = np.array([(j // per) * (per * t + 3 * t) + (j % per) * t for j in range(n)], np.uint64)
            region = 40 * (per * t + 3 * t)
        L = Layout(oracle, n, t)
        dst = gfd_amd.DeviceBuffer(region)
        dst.fill(0xCD)
        ent = (gfd_amd.SGEntry * n)()
        a = np.frombuffer(ent, dtype=np.uint64).reshape(n, 3)
        a[:, 0] = np.uint64(dst.ptr) + offs
        a[:, 1] = L.src_addrs
        a[:, 2] = t
        tt = np.zeros(iters)
        rc = gfd_amd.lib().gfd_bench_submit_direct(poller._h, ctypes.cast(ent, ctypes.c_void_p), n, warmup, iters,
                                                   tt.ctypes.data_as(PD))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        expect = np.full(region, 0xCD, np.uint8)
        toks = L.expected.reshape(n, t)
        for j in range(n):
            expect[int(offs[j]):int(offs[j]) + t] = toks[j]
        if not (dst.download() == expect).all():
            raise SystemExit("PARITY FAILURE: direct with %s destinations" % name)
        out[name] = {"us_p50": round(p50(tt), 2), "GBps": round(gbps(n * t, p50(tt)), 3)}
        log("  8192x4096 direct, scattered destinations (%s): %s" % (name, out[name]))
        del L, dst
    return out


def run_memcpy_n(L, iters, warmup):
    t = np.zeros(iters)
    rc = gfd_amd.lib().gfd_bench_memcpy_per_token(L.dst.ptr, L.src_addrs.ctypes.data, L.n, L.t, warmup, iters,
                                                  t.ctypes.data_as(PD))
    assert rc == 0, gfd_amd.lib().gfd_last_error()
    L.verify("memcpy per token")
    return {"us_p50": round(p50(t), 2), "GBps": round(gbps(L.bytes, p50(t)), 3)}


def run_moe(oracle, iters, warmup, tokens=4096, experts=64, dim=7168):
    """SG-MoE: top-2 of 64 experts per token on the GPU, per-expert row lists
    built on the GPU, then the wave-specialised gather of the routed 14 KiB
    bf16 rows from pinned host memory, with and without the RMSNorm consumer.
    Times are HIP-event kernel times on the launch stream (P50)."""
    L = gfd_amd.lib()
    row_bytes, stride = dim * 2, dim * 4
    vals = oracle.moe_token_values(tokens, dim)
    host = gfd_amd.HostBuffer(tokens * stride)
    host.array[:] = oracle.GAP_BYTE
    host.array.reshape(tokens, stride)[:, :row_bytes] = vals.view(np.uint8).reshape(tokens, row_bytes)
    logits = oracle.moe_logits(tokens, experts)
    offsets, row_token = oracle.moe_lists(oracle.moe_top2(logits), experts)
    weight = oracle.moe_weight(dim)
    n = 2 * tokens
    d_logits = gfd_amd.DeviceBuffer(logits.nbytes)
    d_logits.upload(logits)
    d_top2, d_rows = gfd_amd.DeviceBuffer(n * 4), gfd_amd.DeviceBuffer(n * 4)
    d_off = gfd_amd.DeviceBuffer((experts + 1) * 4)
    d_w = gfd_amd.DeviceBuffer(dim * 2)
    d_w.upload(weight)
    d_dst, d_out, d_err = gfd_amd.DeviceBuffer(n * row_bytes), gfd_amd.DeviceBuffer(n * row_bytes), gfd_amd.DeviceBuffer(4)
    d_err.fill(0)
    st, ea, eb = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    L.gfd_stream_create(ctypes.byref(st))
    L.gfd_event_create(ctypes.byref(ea))
    L.gfd_event_create(ctypes.byref(eb))

    def timed(fn, count):
        out = []
        for i in range(-warmup, count):
            L.gfd_event_record(ea, st)
            fn()
            L.gfd_event_record(eb, st)
            L.gfd_event_synchronize(eb)
            ms = ctypes.c_float(0)
            L.gfd_event_elapsed_ms(ctypes.byref(ms), ea, eb)
            if i >= 0:
                out.append(ms.value * 1000.0)
        return out

    route_us = timed(lambda: gfd_amd.moe_route(d_logits.ptr, tokens, experts, d_top2.ptr, d_off.ptr, d_rows.ptr,
                                               st), iters)
    if not (d_rows.download().view(np.int32) == row_token).all():
        raise SystemExit("PARITY FAILURE: MoE row lists")
    res = {"tokens": tokens, "experts": experts, "rows": n, "row_bytes": row_bytes, "bytes": n * row_bytes,
           "route_and_lists_us_p50": round(p50(route_us), 2)}
    expect = vals[row_token]
    for name, with_norm in (("transfer_only", False), ("overlapped_rmsnorm", True)):
        t = timed(lambda: gfd_amd.sg_gather_rmsnorm(host.ptr, stride, tokens, d_rows.ptr, n, row_bytes, d_dst.ptr,
                                                    d_out.ptr if with_norm else None, d_w.ptr, 1e-6, 0, d_err.ptr,
                                                    st), iters)
        if int(d_err.download().view(np.int32)[0]) != 0:
            raise SystemExit("MoE gather reported an error")
        if not (d_dst.download().view(np.uint16).reshape(n, dim) == expect).all():
            raise SystemExit("PARITY FAILURE: MoE gathered rows (%s)" % name)
        if with_norm:
            ref = oracle.rmsnorm_rows(oracle.bf16_to_f32(expect), oracle.bf16_to_f32(weight), 1e-6)
            got = oracle.bf16_to_f32(d_out.download().view(np.uint16).reshape(n, dim))
            if not np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6):
                raise SystemExit("PARITY FAILURE: MoE RMSNorm outside bf16 tolerance")
        res[name] = {"us_p50": round(p50(t), 2), "GBps": round(gbps(n * row_bytes, p50(t)), 3)}
    # The same workload through SGWarpSpecSession: GPU submitter waves build
    # lists of <= 24 rows from the routing output, the session's transfer
    # waves copy them, its compute waves (3 sharing each list, or the
    # reference's single one) run the RMSNorm.  Timed with HIP
    # events around launch_moe on the stream (the session's per-launch set-up
    # included); the kernel ends itself once every list has landed.
    for name, with_norm, cw in (("session_transfer_only", False, 1),
                                ("session_overlapped_rmsnorm", True, MOE_SESSION_COMPUTE_WAVES),
                                ("session_overlapped_rmsnorm_1_compute_wave", True, 1)):
        sess = gfd_amd.SGWarpSpecSession(num_compute_warps=cw, num_blocks=MOE_SESSION_BLOCKS, idle_limit_ms=10000,
                                         helper_waves=MOE_SESSION_HELPERS)
        try:
            t = []
            for i in range(-warmup, iters):
                sess.reset()
                L.gfd_event_record(ea, st)
                sess.launch_moe(host.ptr, stride, tokens, d_off.ptr, d_rows.ptr, experts, n, row_bytes, d_dst.ptr,
                                d_out.ptr if with_norm else None, d_w.ptr, 1e-6, MOE_SESSION_ROWS_PER_LIST, st)
                L.gfd_event_record(eb, st)
                L.gfd_event_synchronize(eb)
                sess.synchronize(0)
                ms = ctypes.c_float(0)
                L.gfd_event_elapsed_ms(ctypes.byref(ms), ea, eb)
                if i >= 0:
                    t.append(ms.value * 1000.0)
            stt = sess.stats()
            if stt["lists_done"] < experts or stt["units_done"] != n:
                raise SystemExit("MoE session: %s" % stt)
            if not (d_dst.download().view(np.uint16).reshape(n, dim) == expect).all():
                raise SystemExit("PARITY FAILURE: MoE session rows (%s)" % name)
            if with_norm:
                ref = oracle.rmsnorm_rows(oracle.bf16_to_f32(expect), oracle.bf16_to_f32(weight), 1e-6)
                got = oracle.bf16_to_f32(d_out.download().view(np.uint16).reshape(n, dim))
                if not np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6):
                    raise SystemExit("PARITY FAILURE: MoE session RMSNorm outside bf16 tolerance")
            res[name] = {"us_p50": round(p50(t), 2), "GBps": round(gbps(n * row_bytes, p50(t)), 3),
                         "lists": stt["lists_done"], "grid": stt["grid"], "rows_per_list": MOE_SESSION_ROWS_PER_LIST,
                         "compute_waves": cw}
            # One more launch with the per-list device timeline (untimed):
            # where the kernel's time goes around the copies.
            sess.enable_trace(1024)
            sess.reset()
            sess.launch_moe(host.ptr, stride, tokens, d_off.ptr, d_rows.ptr, experts, n, row_bytes, d_dst.ptr,
                            d_out.ptr if with_norm else None, d_w.ptr, 1e-6, MOE_SESSION_ROWS_PER_LIST, st)
            L.gfd_stream_synchronize(st)
            sess.synchronize(0)
            res[name]["timeline"] = session_timeline(*sess.trace(), sess.stats()["lists_done"])
        finally:
            sess.close()
    L.gfd_event_destroy(ea)
    L.gfd_event_destroy(eb)
    L.gfd_stream_destroy(st)
    return res


def session_timeline(lists, blocks, nlists):
    """Summary of one traced SG session launch (device wall clock, us from the
    first workgroup's start): first copy start, last landing, the kernel's
    last wave exit, the spread of the workgroups' last landings, and the mean
    time from a transfer wave looking for a list to its header being read."""
    u = lists[:nlists]
    t0 = int(blocks["start"].min())
    us = lambda x: (np.asarray(x, dtype=np.int64) - t0) / gfd_amd.SG_TRACE_TICKS_PER_US
    last = [float(us(u["landed"][u["block"] == b].max())) for b in range(len(blocks)) if (u["block"] == b).any()]
    return {"first_copy_us": round(float(us(u["ready"].min())), 1),
            "last_landing_us": round(float(us(u["landed"].max())), 1),
            "last_exit_us": round(float(us(blocks["exit"].max())), 1),
            "workgroup_last_landing_us": [round(min(last), 1), round(float(np.median(last)), 1), round(max(last), 1)],
            "claim_to_ready_mean_us": round(float(np.mean(us(u["ready"]) - us(u["claimed"]))), 2)}


def _pmc_pass(exe, counter, workdir, timeout_s):
    """One rocprofv3 --pmc pass over `bench.py --only zc,calib` (5 device-to-
    device copies of 32 MiB, 5 launches of the gather kernel over one
    contiguous 32 MiB pinned range, then 12 launches of the 8192 x 4 KiB
    gather), in its own process group under a time limit.  Per-dispatch
    counter values (KiB): (calibration copies, contiguous calibration
    gathers, gather launches), or a reason string."""
    out = os.path.join(workdir, counter)
    cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "p", "--", sys.executable,
           os.path.join(ROOT, "bench.py"), "--only", "zc,calib", "--cpu-seconds", "0", "--steps", "5", "--warmup", "1"]
    env = dict(os.environ, TMPDIR="/tmp")
    with open(os.path.join(workdir, counter + ".log"), "w") as logf:
        p = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=logf, stderr=subprocess.STDOUT, start_new_session=True)
        try:
            rc = p.wait(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.wait()
            return "%s pass did not finish in %d s" % (counter, timeout_s)
    files = glob.glob(os.path.join(out, "**", "p_counter_collection.csv"), recursive=True)
    if not files:
        return "%s pass wrote no counter file (exit %d)" % (counter, rc)
    copies, contig, gathers = parse_pmc_counters(files[0], counter)
    if len(copies) < 5 or len(contig) < 5 or not gathers:
        return "%s pass: %d calibration copies, %d contiguous gathers, %d gathers counted (exit %d)" % (
            counter, len(copies), len(contig), len(gathers), rc)
    return copies, contig, gathers


def parse_pmc_counters(path, counter):
    """Per-dispatch values of `counter` in a rocprofv3 counter_collection.csv:
    (the calibration copies, the contiguous calibration gathers, the gather
    launches).  The calibration copies run before anything else that could
    use the runtime's copy kernel: the first five dispatches of it.  The
    contiguous gathers are the first five dispatches of the gather kernel
    (they run before the poller exists).  The gathers: the later launches of
    the 8192 x 4 KiB job, the largest grid (the poller's set-up also launches
    the kernel once on 16 bytes)."""
    copies, zc = [], []
    with open(path) as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            name, v = row["Kernel_Name"], float(row["Counter_Value"])
            if "copyBuffer" in name:
                copies.append((int(row["Dispatch_Id"]), v))
            elif "zc_gather_tokens" in name:
                zc.append((int(row["Dispatch_Id"]), int(row["Grid_Size"]), v))
    copies = [v for _, v in sorted(copies)[:5]]
    zc.sort()
    contig, rest = [v for _, _, v in zc[:5]], zc[5:]
    big = max((g for _, g, _ in rest), default=0)
    return copies, contig, [v for _, g, v in rest if g == big]


# Bytes the contiguous calibration gather moves per launch: reads are the
# 32 MiB over the host link plus the 64 KiB page table in HBM, writes the
# 32 MiB into HBM (the same algorithmic bytes as one 8192 x 4 KiB gather).
CALIB_READ_BYTES = (32 << 20) + 8192 * 8
CALIB_WRITE_BYTES = 32 << 20


def measure_traffic(timeout_s=150):
    """HBM-side traffic of one 8192 x 4 KiB zc_gather_tokens launch, measured
    in this run: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) from two
    rocprofv3 --pmc passes, each scaled by the same counter on the same
    kernel reading one contiguous 32 MiB pinned range (bytes known:
    CALIB_READ_BYTES / CALIB_WRITE_BYTES), so host-link reads are calibrated
    on host-link reads.  The factor a 32 MiB device-to-device copy gives is
    kept beside it.  (read_bytes, write_bytes, detail) or (None, None,
    reason)."""
    exe = shutil.which("rocprofv3")
    if not exe:
        return None, None, "rocprofv3 not on PATH"
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        got = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            log("traffic: rocprofv3 --pmc %s pass ..." % counter)
            r = _pmc_pass(exe, counter, td, timeout_s)
            if isinstance(r, str):
                return None, None, r
            got[counter] = r
    detail = {}
    val = {}
    for counter, known in (("FETCH_SIZE", CALIB_READ_BYTES), ("WRITE_SIZE", CALIB_WRITE_BYTES)):
        copies, contig, gathers = got[counter]
        cal = float(np.median(contig))
        scale = known / 1024.0 / cal  # KiB the contiguous gather moves per KiB counted
        copy_scale = 32768.0 / float(np.median(copies))
        val[counter] = float(np.mean(gathers)) * scale * 1024.0
        detail[counter] = {"gather_kib_per_dispatch": round(float(np.mean(gathers)), 2),
                           "gather_dispatches": len(gathers),
                           "contiguous_gather_kib_per_dispatch": round(cal, 2), "scale": round(scale, 5),
                           "copy_kib_per_dispatch": round(float(np.median(copies)), 2),
                           "d2d_copy_scale": round(copy_scale, 5)}
    return int(round(val["FETCH_SIZE"])), int(round(val["WRITE_SIZE"])), detail


def run_offload(oracle, iters, warmup):
    """Offload (HBM -> pinned host, the reverse path): n tokens contiguous in
    HBM written to the seeded 2x-stride slots of a pinned host region by the
    zero-copy scatter kernel, and again as SG lists through a session;
    checked against the oracle's closed form.  The link reference is one
    contiguous device->host hipMemcpyAsync of the same bytes."""
    out = {}
    for n, t in ((8192, 4096), (2048, 65536)):
        nbytes, stride = n * t, 2 * t
        tokens = np.random.default_rng(n + t).integers(0, 256, nbytes, dtype=np.uint8)
        src = gfd_amd.DeviceBuffer(nbytes)
        src.upload(tokens)
        host = gfd_amd.HostBuffer(n * stride)
        host.array[:] = 0xCD
        before = host.array.copy()
        perm = oracle.permutation(n)
        table = gfd_amd.DeviceBuffer(n * 8)
        table.upload(np.uint64(host.ptr) + perm.astype(np.uint64) * np.uint64(stride))
        wall, ev = np.zeros(iters), np.zeros(iters)
        rc = gfd_amd.lib().gfd_bench_zero_copy_scatter_tokens(table.ptr, src.ptr, t, n, warmup, iters,
                                                              wall.ctypes.data_as(PD), ev.ctypes.data_as(PD))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        want_region = oracle.expected_scatter(before, tokens, perm, t, stride)
        assert np.array_equal(host.array, want_region), "offload %dx%d: bytes differ from the oracle" % (n, t)
        contig = gfd_amd.HostBuffer(nbytes)
        tc = np.zeros(iters)
        rc = gfd_amd.lib().gfd_bench_memcpy_contiguous_d2h(contig.ptr, src.ptr, nbytes, 1, warmup, iters,
                                                           tc.ctypes.data_as(PD))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        d2h = gbps(nbytes, p50(tc))
        k_gbps = gbps(nbytes, float(ev.mean()))
        # The same eviction as host-submitted SG lists drained by a running
        # session's transfer waves (lists of 128 tokens; launch until the host
        # has seen every list's done marker).
        host.array[:] = 0xCD
        epl = 128 if n >= 4096 else 32
        ent = gfd_amd.device_sg_entries(src.ptr + np.arange(n, dtype=np.uint64) * np.uint64(t),
                                        host.ptr + perm.astype(np.uint64) * np.uint64(stride), t)
        sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=0, idle_limit_ms=10000)
        sus = sess.bench(ent, epl, warmup=warmup, iters=iters)
        sst = sess.stats()
        sess.close()
        assert np.array_equal(host.array, want_region), "session offload %dx%d: bytes differ" % (n, t)
        out["%dx%d" % (n, t)] = {
            "bytes": nbytes, "zero_copy_scatter": {
                "us_p50": round(p50(wall), 2), "GBps": round(gbps(nbytes, p50(wall)), 3),
                "kernel_us_mean": round(float(ev.mean()), 2), "kernel_GBps": round(k_gbps, 3),
                "of_theoretical": round(k_gbps / PCIE_GEN5_X16_GBPS, 4),
                "of_d2h_contiguous": round(k_gbps / d2h, 4) if d2h else None},
            "sg_session": {"us_p50": round(p50(sus), 2), "GBps": round(gbps(nbytes, p50(sus)), 3),
                           "lists": n // epl, "grid": sst["grid"]},
            "d2h_contiguous_GBps": round(d2h, 3)}
        log("  offload %dx%d: %s" % (n, t, out["%dx%d" % (n, t)]))
        for b in (src, host, table, contig):
            b.free()
    return out


def run_tiled_baseline(oracle, iters, warmup):
    """The poller's tiled mode at the reference's warp-spec example shape
    (examples/07_warp_spec_simple.cu's global-wait baseline: 8192 tokens of
    16 KiB, 128-token tiles, 32-token chunks): one workgroup per tile
    submits its chunks as descriptors and waits for the tile's progress word,
    which the poller raises (copy-engine writes into HBM) after the tile's
    copies; then each token's u32-word checksum.  Timed from the launch until
    the kernel has finished, the poller already running.  The example's
    consumer is RMSNorm + sinf; this one is the checksum used in the tests."""
    tiles, T, C, ts = 64, 128, 32, 16384
    n = tiles * T
    host = gfd_amd.HostBuffer(n * ts)
    host.array[:] = np.random.default_rng(3).integers(0, 256, n * ts, dtype=np.uint8)
    dst = gfd_amd.DeviceBuffer(n * ts)
    sums = gfd_amd.DeviceBuffer(n * 8)
    status = gfd_amd.HostBuffer(64)
    tq = gfd_amd.TiledQueue(tiles, T, C, ts, device_signals=True)
    p = gfd_amd.CpuPollingThread(tq, dst.ptr, host.ptr, host.nbytes, numa_node=-1)
    times = []
    try:
        p.set_tiled_queue(tq)
        assert p.init_copy_engine()
        for i in range(-warmup, iters):
            p.stop()
            tq.reset()
            p.reset_stats()
            status.array.view(np.int32)[0] = 0
            p.start()
            t0 = time.perf_counter()
            gfd_amd.tiled_poller_run(tq, host.ptr, dst.ptr, sums.ptr, status.ptr, whole_tile=False)
            gfd_amd.synchronize()
            t1 = time.perf_counter()
            if int(status.array.view(np.int32)[0]) != 0:
                raise SystemExit("tiled poller baseline: a tile wait timed out")
            if i >= 0:
                times.append((t1 - t0) * 1e6)
        if not (dst.download() == host.array).all():
            raise SystemExit("PARITY FAILURE: tiled poller baseline")
        want = [oracle.u32_word_checksum(host.array[g * ts:(g + 1) * ts]) for g in range(0, n, 97)]
        got = sums.download().view(np.uint64)[::97]
        if [int(x) for x in got] != want:
            raise SystemExit("PARITY FAILURE: tiled poller baseline checksums")
    finally:
        p.stop()
        p.close()
        tq.free()
    return {"bytes": n * ts, "us_p50": round(p50(times), 2), "GBps": round(gbps(n * ts, p50(times)), 3),
            "tiles": tiles, "tokens_per_tile": T, "tokens_per_chunk": C}


def run_sessions(oracle, iters, warmup):
    """Wave-specialised sessions.  WarpSpecSession on linear tiles (token t at
    cpu_src + t*T -> gpu_dst + t*T; T = 128 tokens, automatic chunking, no-op
    consumer), single and double buffered: 8192 x 16 KiB = 128 MiB (the shape
    of the reference's warp-spec example) and 8192 x 4 KiB; the 128 MiB shape
    again with the example's RMSNorm + sinf consumer.  SGWarpSpecSession
    (no-op consumer) on 16384 scattered 4 KiB tokens (2x stride, Fisher-Yates
    order) = 64 MiB in 128 host-submitted lists of 128 entries, timed from
    the launch until the host sees every list's done marker.  Every output is
    compared with the source bytes."""
    out = {}
    for n, t in ((8192, 16384), (8192, 4096)):
        host = gfd_amd.HostBuffer(n * t)
        oracle.fill_tokens(host.array, n, t, t)
        dst = gfd_amd.DeviceBuffer(n * t)
        for db in (False, True):
            dst.fill(0)
            res, kms = gfd_amd.warp_spec_run(host.ptr, dst.ptr, n, t, 128, 0, db, False, 0, iters=warmup + iters)
            if not (dst.download() == host.array).all():
                raise SystemExit("PARITY FAILURE: WarpSpecSession %dx%d db=%d" % (n, t, db))
            us = kms[warmup:] * 1000.0
            key = "warp_spec_%dx%dKB%s" % (n, t // 1024, "_db" if db else "")
            out[key] = {"bytes": n * t, "kernel_us_p50": round(p50(us), 2), "GBps": round(gbps(n * t, p50(us)), 3),
                        "grid": res["grid"], "block": res["block"], "tokens_per_chunk": res["tokens_per_chunk"],
                        "chunks_per_tile": res["chunks_per_tile"]}
            log("  %s: %s" % (key, out[key]))
        del host, dst
    # The reference's warp-spec example with its RMSNorm + sinf consumer
    # (examples/07_warp_spec_simple.cu: 8192 tokens of 4096 floats): seeded
    # standard-normal floats, the per-token result checked against float64.
    n, t = 8192, 16384
    nf = t // 4
    host = gfd_amd.HostBuffer(n * t)
    xs = np.random.default_rng(7).standard_normal(n * nf).astype(np.float32)
    host.array.view(np.float32)[:] = xs
    dst = gfd_amd.DeviceBuffer(n * t)
    outb = gfd_amd.DeviceBuffer(n * 4)
    x64 = xs.reshape(n, nf).astype(np.float64)
    y64 = x64 / np.sqrt(np.mean(x64 * x64, axis=1) + 1e-6)[:, None]
    terms = np.sin(y64) * y64
    want, mag = terms.sum(axis=1), np.abs(terms).sum(axis=1)
    del x64, y64, terms
    # Two tile shapes: 64-token tiles of 8-token chunks, single buffered, on
    # 64 workgroups (the best of a sweep: the consumer's work left after the
    # last chunk lands is smallest), and the example's own 128-token tiles of
    # 32-token chunks, double buffered, on the default grid.
    for key, tile, chunk, db, blocks in (("warp_spec_%dx%dKB_rms_sin" % (n, t // 1024), 64, 8, False, 64),
                                         ("warp_spec_%dx%dKB_rms_sin_example_shape_db" % (n, t // 1024), 128, 32,
                                          True, 0)):
        dst.fill(0)
        outb.fill(0)
        res, kms = gfd_amd.warp_spec_run_rms_sin(host.ptr, dst.ptr, n, t, outb.ptr, tile, chunk, db,
                                                 num_blocks=blocks, iters=warmup + iters)
        got = outb.download().view(np.float32).astype(np.float64)
        if not (dst.download() == host.array).all() or not np.all(np.abs(got - want) <= 1e-4 * mag + 1e-6):
            raise SystemExit("PARITY FAILURE: WarpSpecSession RMSNorm + sinf (%s)" % key)
        us = kms[warmup:] * 1000.0
        out[key] = {"bytes": n * t, "kernel_us_p50": round(p50(us), 2), "GBps": round(gbps(n * t, p50(us)), 3),
                    "grid": res["grid"], "block": res["block"], "tokens_per_tile": tile,
                    "tokens_per_chunk": res["tokens_per_chunk"], "chunks_per_tile": res["chunks_per_tile"],
                    "double_buffer": db}
        log("  %s: %s" % (key, out[key]))
    del host, dst, outb
    n, t, epl = 16384, 4096, 128
    host = gfd_amd.HostBuffer(n * 2 * t)
    oracle.fill_tokens(host.array, n, t, 2 * t)
    perm = oracle.permutation(n)
    dst = gfd_amd.DeviceBuffer(n * t)
    dst.fill(0)
    ent = gfd_amd.device_sg_entries(host.ptr + perm.astype(np.uint64) * np.uint64(2 * t),
                                    dst.ptr + np.arange(n, dtype=np.uint64) * np.uint64(t), t)
    sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=0, idle_limit_ms=10000)
    us = sess.bench(ent, epl, warmup=warmup, iters=iters)
    st = sess.stats()
    sess.close()
    if not (dst.download() == oracle.expected_gather(host.array, perm, t, 2 * t)).all():
        raise SystemExit("PARITY FAILURE: SGWarpSpecSession 16384x4KB")
    out["sg_16384x4KB_lists128"] = {"bytes": n * t, "us_p50": round(p50(us), 2), "GBps": round(gbps(n * t, p50(us)), 3),
                                    "grid": st["grid"], "entries_per_list": epl}
    log("  sg_16384x4KB_lists128: %s" % out["sg_16384x4KB_lists128"])
    return out


def run_helper_waves(oracle, iters, warmup):
    """Transfer helper waves at small grids (1, 4 and 8 workgroups, the block
    counts the reference's own tests use): WarpSpecSession 8192 x 16 KiB and
    SGWarpSpecSession 16384 x 4 KiB scattered in lists of 512, each without
    helpers and with 3.  Outputs are compared with the source bytes."""
    out = {}
    n, t = 8192, 16384
    host = gfd_amd.HostBuffer(n * t)
    oracle.fill_tokens(host.array, n, t, t)
    dst = gfd_amd.DeviceBuffer(n * t)
    for blocks in (1, 4, 8):
        for h in (0, 3):
            dst.fill(0)
            res, kms = gfd_amd.warp_spec_run(host.ptr, dst.ptr, n, t, 128, 0, False, False, blocks,
                                             iters=warmup + iters, helper_waves=h)
            if not (dst.download() == host.array).all():
                raise SystemExit("PARITY FAILURE: WarpSpecSession blocks=%d helpers=%d" % (blocks, h))
            us = kms[warmup:] * 1000.0
            key = "warp_spec_%dx%dKB_blocks%d_helpers%d" % (n, t // 1024, blocks, h)
            out[key] = {"kernel_us_p50": round(p50(us), 2), "GBps": round(gbps(n * t, p50(us)), 3),
                        "block": res["block"]}
            log("  %s: %s" % (key, out[key]))
    del host, dst
    n, t, epl = 16384, 4096, 512
    host = gfd_amd.HostBuffer(n * 2 * t)
    oracle.fill_tokens(host.array, n, t, 2 * t)
    perm = oracle.permutation(n)
    dst = gfd_amd.DeviceBuffer(n * t)
    ent = gfd_amd.device_sg_entries(host.ptr + perm.astype(np.uint64) * np.uint64(2 * t),
                                    dst.ptr + np.arange(n, dtype=np.uint64) * np.uint64(t), t)
    want = oracle.expected_gather(host.array, perm, t, 2 * t)
    for blocks in (1, 4, 8):
        for h in (0, 3):
            dst.fill(0)
            sess = gfd_amd.SGWarpSpecSession(num_compute_warps=1, num_blocks=blocks, idle_limit_ms=10000,
                                            helper_waves=h)
            us = sess.bench(ent, epl, warmup=max(1, warmup // 5), iters=max(3, iters // 5))
            sess.close()
            if not (dst.download() == want).all():
                raise SystemExit("PARITY FAILURE: SGWarpSpecSession blocks=%d helpers=%d" % (blocks, h))
            key = "sg_16384x4KB_lists512_blocks%d_helpers%d" % (blocks, h)
            out[key] = {"us_p50": round(p50(us), 2), "GBps": round(gbps(n * t, p50(us)), 3)}
            log("  %s: %s" % (key, out[key]))
    return out


TRACE_NAMES = {1: "batch_first_read", 2: "flush", 3: "copies_issued", 4: "done_published", 5: "gap_flush",
               7: "chunk_copy_issued", 8: "direct_end", 9: "gather_entry", 10: "gather_idle",
               11: "gather_published", 12: "gather_first_slice", 13: "gather_built", 14: "zc_kernel_launched",
               15: "zc_done_seen", 16: "zc_checked"}


def _phase_medians(rows):
    """rows: list of {phase: us}; median per phase over the rows that have it."""
    keys = []
    for r in rows:
        for k in r:
            if k not in keys:
                keys.append(k)
    out = {}
    for k in keys:
        v = [r[k] for r in rows if k in r]
        out[k] = round(float(np.median(v)), 2)
    return dict(sorted(out.items(), key=lambda kv: kv[1]))


def _call_phases(tr, cp, t0, t1):
    """Phase times (us after t0) of one call from the poller trace `tr` and
    the SDMA copy timeline `cp`, both on CLOCK_MONOTONIC ns."""
    ph = {}
    for ev in tr[(tr["t_ns"] >= t0) & (tr["t_ns"] <= t1)]:
        name = TRACE_NAMES.get(int(ev["kind"]))
        if name is None:
            continue
        us = (int(ev["t_ns"]) - t0) / 1e3
        if name + "_first" not in ph:
            ph[name + "_first"] = us
        ph[name + "_last"] = us
    c = cp[(cp["start_ns"] >= t0) & (cp["end_ns"] <= t1)]
    if len(c):
        ph["sdma_first_start"] = (int(c["start_ns"].min()) - t0) / 1e3
        ph["sdma_last_end"] = (int(c["end_ns"].max()) - t0) / 1e3
        ph["sdma_copies"] = float(len(c))
    ph["return"] = (t1 - t0) / 1e3
    return ph


def run_timeline(oracle, calls=30):
    """Where the time of one call goes, for GFD Direct and GFD Queue at
    2048 x {512, 1024, 2048} B and 8192 x 4 KiB: the poller's trace events
    and the SDMA copy timeline of `calls` back-to-back calls, as the median
    time of each phase after the call starts (us).  Direct: from entry into
    submit_direct to its return.  Queue: from the host's launch of the
    submit kernel to the return of the stream synchronisation after the wait
    kernel.  Every call's output is compared with the oracle."""
    L_ = gfd_amd.lib()
    out = {"calls": calls}
    shapes = [(2048, 512), (2048, 1024), (2048, 2048), (8192, 4096)]
    direct = gfd_amd.CpuPollingThread(None, None, None, 8192 * 4096 * 2, numa_node=-1)
    assert direct.init_direct_ce(), "init_direct_ce failed"
    for n, t in shapes:
        L = Layout(oracle, n, t)
        routes = [("", DIRECT_ZC_MAX)] + ([("_staged", 0)] if n * t <= DIRECT_ZC_MAX else [])
        for suffix, zc_max in routes:
            direct.set_direct_zero_copy_max_bytes(zc_max)
            for _ in range(10):
                assert direct.submit_direct(L.entries, L.n) > 0
            direct.set_trace(True)
            direct.set_copy_timing(True)
            direct.read_trace()
            direct.read_copy_times()
            win = []
            for _ in range(calls):
                a = time.monotonic_ns()
                assert direct.submit_direct(L.entries, L.n) > 0
                win.append((a, time.monotonic_ns()))
            tr, cp = direct.read_trace(), direct.read_copy_times()
            direct.set_trace(False)
            direct.set_copy_timing(False)
            L.verify("direct (timeline)")
            rows = []
            for a, b in win:
                begin = tr[(tr["kind"] == 6) & (tr["t_ns"] >= a) & (tr["t_ns"] <= b)]
                t0 = int(begin["t_ns"][0]) if len(begin) else a
                rows.append(_call_phases(tr, cp[cp["path"] == 1], t0, b))
            key = "direct%s_%dx%d" % (suffix, n, t)
            out[key] = _phase_medians(rows)
            log("  timeline %s: %s" % (key, out[key]))
        direct.set_direct_zero_copy_max_bytes(DIRECT_ZC_MAX)
        del L
    direct.close()

    for worker in (False, True):
        out.update(_queue_timeline(oracle, shapes if not worker else shapes[:3], calls, worker))
    return out


def _queue_timeline(oracle, shapes, calls, worker):
    """The Queue half of run_timeline; with `worker`, the poller's persistent
    zero-copy worker copies the batches (keys queue_worker_<n>x<t>)."""
    L_ = gfd_amd.lib()
    out = {}
    q = gfd_amd.DescriptorQueue()
    p = gfd_amd.CpuPollingThread(q, None, None, 8192 * 4096 * 2, numa_node=-1)
    assert p.init_copy_engine(), "queue poller init failed"
    if worker:
        p.set_zero_copy_worker(True)
    p.start()
    st = ctypes.c_void_p()
    L_.gfd_stream_create(ctypes.byref(st))
    status = gfd_amd.HostBuffer(64, gfd_amd.HOST_COHERENT)
    base = 0
    try:
        for n, t in shapes:
            L = Layout(oracle, n, t)
            rows = []
            for i in range(10 + calls):
                if i == 10:
                    p.set_trace(True)
                    p.set_copy_timing(True)
                    p.read_trace()
                    p.read_copy_times()
                status.array.view(np.int32)[0] = -1
                a = time.monotonic_ns()
                assert L_.gfd_queue_submit_tokens(q.ptr, L.tokens.ptr, L.dst.ptr, n, t, base, st) == 0
                base += n
                assert L_.gfd_queue_wait(q.ptr, base, 10_000_000, status.ptr, st) == 0
                assert L_.gfd_stream_synchronize(st) == 0
                b = time.monotonic_ns()
                assert int(status.array.view(np.int32)[0]) == 0, "queue wait timed out"
                if i >= 10:
                    rows.append((a, b))
            tr, cp = p.read_trace(), p.read_copy_times()
            p.set_trace(False)
            p.set_copy_timing(False)
            L.verify("queue (timeline)")
            key = "queue%s_%dx%d" % ("_worker" if worker else "", n, t)
            out[key] = _phase_medians([_call_phases(tr, cp[cp["path"] == 0], a, b) for a, b in rows])
            log("  timeline %s: %s" % (key, out[key]))
            del L
    finally:
        L_.gfd_stream_destroy(st)
        p.stop()
        p.close()
        q.free()
    return out


def first_call_latency(oracle):
    """A fresh poller's first submit_direct (256 x 4 KiB scattered, 1 MiB),
    then its second: the one-off set-up cost a caller pays on first use."""
    L = Layout(oracle, 256, 4096)
    t_init = time.monotonic_ns()
    p = gfd_amd.CpuPollingThread(None, None, None, L.n * L.stride, numa_node=-1)
    assert p.init_direct_ce(), "init_direct_ce failed"
    init_us = (time.monotonic_ns() - t_init) / 1e3
    first = p.submit_direct(L.entries, L.n)
    second = p.submit_direct(L.entries, L.n)
    p.close()
    L.verify("direct (first call)")
    return {"init_direct_ce_us": round(init_us, 1), "first_call_us": round(first, 2),
            "second_call_us": round(second, 2)}


class QueueRig:
    def __init__(self, region_bytes, worker=False):
        self.q = gfd_amd.DescriptorQueue()
        self.p = gfd_amd.CpuPollingThread(self.q, None, None, region_bytes, numa_node=-1)
        assert self.p.init_copy_engine(), "queue poller init failed"
        if worker:
            self.p.set_zero_copy_worker(True)
        self.p.start()
        self.base = ctypes.c_uint64(0)

    def run(self, L, iters, warmup):
        t = np.zeros(iters)
        rc = gfd_amd.lib().gfd_bench_queue(self.q.ptr, L.tokens.ptr, L.dst.ptr, L.n, L.t, ctypes.byref(self.base),
                                           warmup, iters, 10_000_000, t.ctypes.data_as(PD))
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        L.verify("queue")
        out = {"us_p50": round(p50(t), 2), "GBps": round(gbps(L.bytes, p50(t)), 3),
               "descriptors_per_s": round(L.n / (p50(t) * 1e-6))}
        w = self.p.zero_copy_worker_stats()
        if w["jobs"]:
            out["worker"] = w
        # SDMA timeline over a few more rounds (after the timed loop).
        self.p.set_copy_timing(True)
        t2 = np.zeros(5)
        t0 = self.p.copy_clock_ns()
        rc = gfd_amd.lib().gfd_bench_queue(self.q.ptr, L.tokens.ptr, L.dst.ptr, L.n, L.t, ctypes.byref(self.base),
                                           0, 5, 10_000_000, t2.ctypes.data_as(PD))
        t1 = self.p.copy_clock_ns()
        copies = self.p.read_copy_times()
        self.p.set_copy_timing(False)
        assert rc == 0, gfd_amd.lib().gfd_last_error()
        occ = sdma_occupancy(copies[copies["path"] == 0], t0, t1)
        if occ:
            occ["rounds"] = 5
        out["sdma"] = occ
        return out

    def close(self):
        self.p.stop()
        self.p.close()
        self.q.free()


def flat_metric_fields(roofline, results, r_moe, r_worker=None):
    """The metric's figures as flat scalars in `roofline` (a record that keeps
    only scalar fields keeps these): per layout, Direct, the zero-copy kernel,
    Queue and per-token copies (us, GB/s, fraction of 63.02 GB/s); the
    Direct / per-token ratio at 4 KiB (target >= 10); the Direct call's SDMA
    occupancy; and config 5 with and without its routing step."""
    for r in results:
        if not r:
            continue
        tag = "%dx%s" % (r["tokens"], ("%dKB" % (r["token_bytes"] // 1024)) if r["token_bytes"] >= 1024
                         else "%dB" % r["token_bytes"])
        for key, name in (("direct", "direct"), ("zero_copy", "zc"), ("queue", "queue"),
                          ("queue_worker", "queue_worker"), ("memcpy_per_token", "memcpy_per_token")):
            m = r.get(key)
            if not m:
                continue
            roofline["%s_%s_us" % (name, tag)] = m["us_p50"]
            roofline["%s_%s_GBps" % (name, tag)] = m["GBps"]
            roofline["%s_%s_frac" % (name, tag)] = round(m["GBps"] / PCIE_GEN5_X16_GBPS, 4)
            if key == "zero_copy":
                roofline["zc_%s_kernel_GBps" % tag] = m["kernel_GBps"]
            if key == "direct" and "route" in m:
                roofline["direct_%s_route" % tag] = m["route"]
        d, c = r.get("direct"), r.get("memcpy_per_token")
        if d and c:
            roofline["direct_over_memcpy_per_token_%s" % tag] = round(c["us_p50"] / d["us_p50"], 2)
        sd = (d or {}).get("sdma")
        if sd:
            roofline["direct_sdma_%s_GBps_over_call" % tag] = round(r["bytes"] / (sd["window_us"] * 1e3), 3)
            roofline["direct_sdma_%s_GBps_while_busy" % tag] = sd["link_GBps_while_busy"]
            roofline["direct_sdma_%s_busy_frac" % tag] = sd["busy_frac_any"]
            roofline["direct_sdma_%s_first_copy_us" % tag] = sd["first_copy_start_us"]
    for key, m in (r_worker or {}).items():
        if isinstance(m, dict) and "us_p50" in m:
            roofline["direct_worker_%s_us" % key] = m["us_p50"]
            roofline["direct_worker_%s_GBps" % key] = m["GBps"]
            if "reference_us" in m:
                roofline["direct_worker_%s_reference_us" % key] = m["reference_us"]
    if r_moe:
        route = r_moe["route_and_lists_us_p50"]
        roofline["moe_route_and_lists_us"] = route
        for key, name in (("transfer_only", "moe_bespoke_transfer"), ("overlapped_rmsnorm", "moe_bespoke_rmsnorm"),
                          ("session_transfer_only", "moe_session_transfer"),
                          ("session_overlapped_rmsnorm", "moe_session_rmsnorm")):
            m = r_moe.get(key)
            if not m:
                continue
            roofline[name + "_us"] = m["us_p50"]
            roofline[name + "_GBps"] = m["GBps"]
            roofline[name + "_with_route_GBps"] = round(gbps(r_moe["bytes"], m["us_p50"] + route), 3)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=15)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="",
                    help="comma list: peak,zc,direct,memcpy,queue,cpu,kv,small,moe,sessions,scattered,offload,worker,"
                         "firstcall,sizes,pmc,helpers,timeline (helpers and timeline are not in the default run; pmc: "
                         "the two rocprofv3 --pmc passes behind roofline.traffic, with zc) "
                         "(calib: add a 32 MiB D2D copy)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this path has no multi-GPU step (each GPU gathers over its own "
              "PCIe link); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    only = set(x for x in args.only.split(",") if x)
    want = (lambda k: not only or k in only)
    K, W = args.steps, args.warmup

    import oracle

    info = host_info()
    log("host:", info)
    result = {}
    cpu = None
    if want("cpu") and args.cpu_seconds > 0:
        log("cpu baseline ...")
        cpu = cpu_baseline(oracle, args.cpu_seconds, info)
        log("cpu baseline:", cpu)

    assert gfd_amd.device_count() > 0, "no GPU visible"
    gfd_amd.lib().gfd_set_device(0)

    if "calib" in only:
        # Reference kernels for the FETCH_SIZE / WRITE_SIZE counters: a device
        # to device copy of 32 MiB (the runtime's blit kernel), 5 launches;
        # then the gather kernel itself over one contiguous 32 MiB pinned range
        # (8192 tokens of 4 KiB in order), 5 launches: the same algorithmic
        # bytes as the scattered gather, read over the host link.
        a = gfd_amd.DeviceBuffer(32 << 20)
        b = gfd_amd.DeviceBuffer(32 << 20)
        a.fill(1)
        for _ in range(5):
            gfd_amd.lib().gfd_memcpy_d2d(b.ptr, a.ptr, 32 << 20)
        gfd_amd.synchronize()
        contig = gfd_amd.HostBuffer(32 << 20)
        contig.array[:] = 7
        tab = gfd_amd.DeviceBuffer(8192 * 8)
        tab.upload(np.uint64(contig.ptr) + np.arange(8192, dtype=np.uint64) * np.uint64(4096))
        for _ in range(5):
            gfd_amd.zero_copy_gather_tokens(tab.ptr, b.ptr, 4096, 8192)
        gfd_amd.synchronize()
        if not (b.download() == 7).all():
            raise SystemExit("PARITY FAILURE: contiguous calibration gather")
        log("calibration done: 5 x 32 MiB device-to-device copies, 5 contiguous 32 MiB gathers")

    peak = {}
    if want("peak"):
        log("contiguous peak ...")
        peak = bench_peak(128 << 20, K, W)
        log("peak:", peak)
    peak_meas = max(v for v in peak.values() if isinstance(v, float)) if peak else None

    main_cfg = (8192, 4096)
    kv_cfg = (2048, 65536)
    small = [(2048, 512), (2048, 1024), (2048, 2048)]
    region_max = 2048 * 65536 * 2
    cfgs = [main_cfg] + ([kv_cfg] if want("kv") else []) + (small if want("small") else [])
    res = {c: {"tokens": c[0], "token_bytes": c[1], "bytes": c[0] * c[1]} for c in cfgs}

    # Phase 1: zero-copy kernel, GFD Direct and per-token copies.  Only the
    # direct poller's gather workers exist (the queue poller is not created
    # yet), so the two pollers never compete for the host cores.
    direct = gfd_amd.CpuPollingThread(None, None, None, region_max, numa_node=-1)
    assert direct.init_direct_ce(), "init_direct_ce failed"
    dinfo = direct.info()
    log("direct poller:", dinfo)
    for n, t in cfgs:
        L = Layout(oracle, n, t)
        r = res[(n, t)]
        if want("zc"):
            r["zero_copy"] = run_zero_copy(L, K, W)
            log("  %dx%d zero-copy: %s" % (n, t, r["zero_copy"]))
        if want("direct"):
            r["direct"] = run_direct(direct, L, K, W)
            log("  %dx%d direct: %s" % (n, t, r["direct"]))
            r["direct"]["sdma"] = direct_timeline(direct, L)
            log("  %dx%d direct SDMA timeline: %s" % (n, t, r["direct"]["sdma"]))
        if want("memcpy"):
            r["memcpy_per_token"] = run_memcpy_n(L, max(5, K // 5), 2)
            log("  %dx%d memcpy(N): %s" % (n, t, r["memcpy_per_token"]))
        del L
    r_scat = None
    if want("direct") and want("scattered"):
        r_scat = run_direct_scattered(oracle, direct, K, W)
    r_sizes = None
    if want("direct") and want("sizes"):
        log("direct at the reference's published token counts ...")
        r_sizes = run_direct_sizes(oracle, direct, K, W)
    r_short = None
    if want("direct") and want("short"):
        log("short lists of large entries ...")
        r_short = run_short_lists(oracle, direct, K, W)
    direct.close()

    r_worker = None
    if want("worker"):
        log("submit_direct through the persistent zero-copy worker ...")
        r_worker = run_worker_direct(oracle, K, W)

    r_sessions = None
    if want("sessions"):
        log("wave-specialised sessions ...")
        r_sessions = run_sessions(oracle, K, W)
        log("poller tiled mode (the example's global-wait baseline) ...")
        r_sessions["tiled_poller_baseline_8192x16KB"] = run_tiled_baseline(oracle, max(5, K // 5), 2)
        log("  tiled poller baseline: %s" % r_sessions["tiled_poller_baseline_8192x16KB"])

    r_timeline = None
    if "timeline" in only:
        log("per-call timelines (Direct, Queue) ...")
        r_timeline = run_timeline(oracle)

    r_first = None
    if want("firstcall"):
        r_first = first_call_latency(oracle)
        log("first submit_direct of a fresh poller: %s" % r_first)

    r_helpers = None
    if "helpers" in only:
        log("transfer helper waves at 1/4/8 workgroups ...")
        r_helpers = run_helper_waves(oracle, K, W)

    r_offload = None
    if want("offload"):
        log("offload (HBM -> pinned host) ...")
        r_offload = run_offload(oracle, K, W)

    r_moe = None
    if want("moe"):
        log("SG-MoE 4096 x 7168 bf16, top-2 of 64 ...")
        r_moe = run_moe(oracle, K, W)
        log("  sg-moe: %s" % r_moe)

    # Phase 2: GFD Queue (GPU-submitted descriptors + CPU poller).
    if want("queue"):
        queue = QueueRig(region_max)
        for n, t in cfgs:
            L = Layout(oracle, n, t)
            res[(n, t)]["queue"] = queue.run(L, K, W)
            log("  %dx%d queue: %s" % (n, t, res[(n, t)]["queue"]))
            del L
        queue.close()
        if want("worker"):
            # The same descriptors with the persistent zero-copy worker copying
            # the batches of at most 4 MiB (config 4).
            queue = QueueRig(region_max, worker=True)
            for n, t in small if want("small") else []:
                L = Layout(oracle, n, t)
                res[(n, t)]["queue_worker"] = queue.run(L, K, W)
                log("  %dx%d queue through the worker: %s" % (n, t, res[(n, t)]["queue_worker"]))
                del L
            queue.close()
    r_main = res[main_cfg]
    r_kv = res.get(kv_cfg)
    r_small = [res[c] for c in small if c in res]

    def frac(v):
        return {"of_theoretical": round(v / PCIE_GEN5_X16_GBPS, 4),
                "of_measured": round(v / peak_meas, 4) if peak_meas else None}

    head = r_main.get("direct") or r_main.get("zero_copy") or {}
    value = head.get("GBps", 0.0)
    zc = r_main.get("zero_copy")
    roofline = None
    if zc:
        ach = zc["kernel_GBps"]
        alg_read = r_main["bytes"] + 8 * r_main["tokens"]  # tokens over the host link + the page table
        alg_write = r_main["bytes"]                         # tokens into HBM
        # traffic: bytes through the L2's memory interface per launch (reads: host-link reads + page
        # table; writes: HBM), measured in this run by two rocprofv3 --pmc passes when the default
        # run asks for them; algorithmic_traffic is the same sum of the algorithmic bytes.
        rd, wr, tdetail = (None, None, "not measured in this run (bench.py --only without pmc)")
        if want("pmc"):
            rd, wr, tdetail = measure_traffic()
            log("traffic:", rd, wr, tdetail)
        if rd is not None:
            source = ("rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes of this run, each scaled by the same kernel "
                      "reading one contiguous 32 MiB pinned range")
        else:
            source = ("profiles/zc_gather_tokens_8192x4KB.md (an earlier run's --pmc passes); this run: %s"
                      % tdetail)
            rd, wr, tdetail = ZC_TRAFFIC_8192x4KB["read_bytes"], ZC_TRAFFIC_8192x4KB["write_bytes"], None
        meas = rd + wr
        roofline = {"bound": "pcie", "kernel": "zc_gather_tokens", "achieved": ach,
                    "peak": round(PCIE_GEN5_X16_GBPS, 2), "unit": "GB/s",
                    "frac": round(ach / PCIE_GEN5_X16_GBPS, 4),
                    "traffic": meas,
                    "traffic_source": source,
                    "algorithmic_traffic": alg_read + alg_write,
                    "traffic_over_algorithmic": round(meas / (alg_read + alg_write), 4),
                    "traffic_detail": dict(read_bytes=rd, write_bytes=wr, algorithmic_read=alg_read,
                                           algorithmic_write=alg_write,
                                           read_over_algorithmic=round(rd / alg_read, 4),
                                           write_over_algorithmic=round(wr / alg_write, 4),
                                           counters=tdetail),
                    "peak_measured": peak_meas,
                    "frac_of_measured": round(ach / peak_meas, 4) if peak_meas else None,
                    "algorithmic_bytes_per_launch": r_main["bytes"],
                    "hbm_write_GBps": ach, "hbm_write_frac": round(ach / 8000.0, 5)}
        dsd = (r_main.get("direct") or {}).get("sdma")
        if dsd:
            # The Direct path's own bound: SDMA copies over the same link.  achieved = the call's
            # bytes over its whole window; while_busy = over the time any engine is copying.
            roofline["direct_sdma"] = {
                "achieved": round(r_main["bytes"] / (dsd["window_us"] * 1e3), 3),
                "link_GBps_while_busy": dsd["link_GBps_while_busy"], "busy_frac_any": dsd["busy_frac_any"],
                "frac": round(r_main["bytes"] / (dsd["window_us"] * 1e3) / PCIE_GEN5_X16_GBPS, 4),
                "frac_while_busy": round(dsd["link_GBps_while_busy"] / PCIE_GEN5_X16_GBPS, 4),
                "first_copy_start_us": dsd["first_copy_start_us"], "copies_per_call": dsd["copies_per_call"],
                "sdma_bytes_per_call": dsd["sdma_bytes_per_call"]}
    for r in [r_main, r_kv] + r_small:
        if not r:
            continue
        for k in ("zero_copy", "direct", "queue", "queue_worker", "memcpy_per_token"):
            if k in r:
                r[k].update(frac(r[k]["GBps"]))
    if roofline is not None:
        flat_metric_fields(roofline, [r_main, r_kv] + r_small, r_moe, r_worker)
    result = {
        "metric": METRIC, "value": round(value, 3), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(head.get("us_p50", 0.0) / 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8",
        "data": "synthetic: xorshift64 token bytes (seed 0x9E3779B97F4A7C15), 2x stride, 0xEE gaps, "
                "Fisher-Yates order (seed 0xD1B54A32D192ED03); every method's output memcmp-checked",
        "config": {"workload": "GFD Direct (CpuPollingThread::submit_direct): 8192 x 4KiB scattered pinned-host "
                               "tokens -> contiguous HBM (32 MiB), P50 of %d" % K,
                   "tokens": 8192, "token_bytes": 4096, "stride": "2x", "parallelism": "single GPU"},
        "pcie_peak": {"theoretical_GBps": round(PCIE_GEN5_X16_GBPS, 2), "measured_contiguous_GBps": peak},
        "roofline": roofline, "cpu_baseline": cpu,
        "results_8192x4KB": r_main, "results_2048x64KB": r_kv, "results_small": r_small, "results_sg_moe": r_moe,
        "results_sessions": r_sessions,
        "results_direct_scattered_dst_8192x4KB": r_scat,
        "results_direct_sizes": r_sizes,
        "results_short_lists": r_short,
        "results_offload": r_offload,
        "results_worker_direct": r_worker,
        "results_helper_waves": r_helpers,
        "results_timeline": r_timeline,
        "first_call_direct_256x4KB": r_first,
        "direct_setup": {k: dinfo[k] for k in ("numa_node", "num_gather_workers", "worker_cpus", "poller_cpu",
                                               "num_ce_channels", "direct_chunk_bytes", "gather_slice_bytes")},
        "host": info,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
