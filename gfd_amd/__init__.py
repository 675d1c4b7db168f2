"""gfd_amd — MI355X-native GFD: scattered host-to-HBM gather.

Python mirror of the reference's host API (``include/gfd/cpu_polling.h``,
``include/gfd/staging_pool.h``), bound over the C-ABI in
``include/gfd_capi.h`` (``libgfd_amd.so``).  The library must be built
(``python -m gfd_amd.builder``); importing this package without it raises
ImportError — there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgfd_amd.so")

__all__ = [
    "lib", "SGEntry", "HostBuffer", "DeviceBuffer", "CpuPollingThread", "StagingPool",
    "DescriptorQueue", "zero_copy_gather_tokens", "zero_copy_gather", "GfdError",
    "HOST_DEFAULT", "HOST_COHERENT", "HOST_NONCOHERENT", "HOST_NUMA_USER", "QUEUE_SIZE",
]

HOST_DEFAULT, HOST_COHERENT, HOST_NONCOHERENT, HOST_NUMA_USER = 0, 1, 2, 4
QUEUE_SIZE = 16384
MAX_BATCH_SIZE = 8192
BATCH_THRESHOLD = 4096
BATCH_THRESHOLD_SMALL = 1024
FLAG_LAST_IN_BATCH, FLAG_URGENT, FLAG_LAST_IN_TILE, FLAG_LAST_CHUNK_IN_TILE = 1, 2, 4, 8


class GfdError(RuntimeError):
    pass


class SGEntry(ctypes.Structure):
    """gfd_sg_entry / gfd::SGEntry: 24 bytes {u64 dst, u64 src, u64 size}."""

    _fields_ = [("dst", ctypes.c_uint64), ("src", ctypes.c_uint64), ("size", ctypes.c_uint64)]


class TokenInfo(ctypes.Structure):
    _fields_ = [("cpu_addr", ctypes.c_uint64), ("token_id", ctypes.c_uint32), ("expert_id", ctypes.c_uint32)]


class PollerStats(ctypes.Structure):
    _fields_ = [
        ("descriptors_processed", ctypes.c_uint64), ("batches_submitted", ctypes.c_uint64),
        ("coalesced_entries", ctypes.c_uint64), ("staging_batches", ctypes.c_uint64),
        ("total_bytes_copied", ctypes.c_double), ("gather_us", ctypes.c_uint64),
        ("dma_wait_us", ctypes.c_uint64), ("dma_submit_us", ctypes.c_uint64),
        ("queue_read_us", ctypes.c_uint64),
    ]


class PollerInfo(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int), ("numa_node", ctypes.c_int), ("num_gather_workers", ctypes.c_int),
        ("poller_cpu", ctypes.c_int), ("worker_cpus", ctypes.c_int * 16), ("num_ce_channels", ctypes.c_int),
        ("num_staging_buffers", ctypes.c_int), ("staging_buffer_size", ctypes.c_uint64),
        ("direct_chunk_bytes", ctypes.c_uint64), ("gather_slice_bytes", ctypes.c_uint64),
        ("staging_pool_set", ctypes.c_int), ("running", ctypes.c_int),
    ]


class DeviceSGEntry(ctypes.Structure):
    """gfd_device_sg_entry / gfd::DeviceSGEntry: 24 bytes {u64 src, u64 dst, u32 size, u32 tag}."""

    _fields_ = [("src", ctypes.c_uint64), ("dst", ctypes.c_uint64), ("size", ctypes.c_uint32),
                ("tag", ctypes.c_uint32)]


DEVICE_SG_ENTRY_DTYPE = np.dtype([("src", np.uint64), ("dst", np.uint64), ("size", np.uint32), ("tag", np.uint32)])


class SessionResult(ctypes.Structure):
    """gfd_session_result: a session's get_stats() plus kernel-reported counters."""

    _fields_ = [("units_done", ctypes.c_uint64), ("bytes", ctypes.c_uint64), ("lists_done", ctypes.c_uint64),
                ("error_bits", ctypes.c_uint64), ("elapsed_ms", ctypes.c_double), ("grid", ctypes.c_int),
                ("block", ctypes.c_int), ("tokens_per_chunk", ctypes.c_int), ("chunks_per_tile", ctypes.c_int),
                ("helper_waves", ctypes.c_int)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


MAX_TILES = 1024
MAX_SG_LISTS = 512
# Bits of an SG session's error word (include/gfd/sg_task_queue.h).
SG_ERR_RING_WAIT = 4
SG_ERR_LIST_WAIT = 32
SG_ERR_DEADLINE = 64
# offsetof(gfd::SGTaskQueue, list_alloc_idx) (static_assert in sg_poller_kernels.hip).
SG_QUEUE_LIST_ALLOC_IDX_OFFSET = 409600
MAX_SG_POOL_ENTRIES = 16384
SG_FLAG_NONE, SG_FLAG_HOST_SUBMITTED = 0, 1


COPY_TIME_DTYPE = np.dtype([("seq", np.uint64), ("bytes", np.uint64), ("start_ns", np.uint64), ("end_ns", np.uint64),
                            ("channel", np.uint32), ("engine", np.uint32), ("path", np.uint32), ("_pad", np.uint32)])

TRACE_DTYPE = np.dtype([("t_ns", np.uint64), ("kind", np.uint32), ("a", np.uint32), ("b", np.uint64)])
TRACE_KINDS = {1: "batch_first", 2: "flush", 3: "issued", 4: "done", 5: "gap_flush", 6: "direct_begin",
               7: "chunk", 8: "direct_end", 9: "gather_entry", 10: "gather_idle", 11: "gather_published",
               12: "gather_first_slice", 13: "gather_built", 14: "zc_launch", 15: "zc_done", 16: "zc_checked"}

_lib = None
_SIGNATURES = {}


def _declare(L):
    c_int, c_u32, c_u64, c_sz, vp, c_dbl = (ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t,
                                             ctypes.c_void_p, ctypes.c_double)
    pvp = ctypes.POINTER(ctypes.c_void_p)
    pd = ctypes.POINTER(ctypes.c_double)
    sig = {
        "gfd_version": ([], ctypes.c_char_p),
        "gfd_last_error": ([], ctypes.c_char_p),
        "gfd_device_count": ([ctypes.POINTER(c_int)], c_int),
        "gfd_set_device": ([c_int], c_int),
        "gfd_device_synchronize": ([], c_int),
        "gfd_host_alloc": ([pvp, c_sz, ctypes.c_uint], c_int),
        "gfd_host_free": ([vp], c_int),
        "gfd_device_alloc": ([pvp, c_sz], c_int),
        "gfd_device_free": ([vp], c_int),
        "gfd_memcpy_h2d": ([vp, vp, c_sz], c_int),
        "gfd_memcpy_d2h": ([vp, vp, c_sz], c_int),
        "gfd_memcpy_d2d": ([vp, vp, c_sz], c_int),
        "gfd_memset_device": ([vp, c_int, c_sz], c_int),
        "gfd_stream_create": ([pvp], c_int),
        "gfd_stream_destroy": ([vp], c_int),
        "gfd_stream_synchronize": ([vp], c_int),
        "gfd_event_create": ([pvp], c_int),
        "gfd_event_destroy": ([vp], c_int),
        "gfd_event_record": ([vp, vp], c_int),
        "gfd_event_synchronize": ([vp], c_int),
        "gfd_event_elapsed_ms": ([ctypes.POINTER(ctypes.c_float), vp, vp], c_int),
        "gfd_poller_create": ([vp, vp, vp, c_sz, c_int, c_int, c_int, c_int, c_int, c_int], vp),
        "gfd_poller_destroy": ([vp], None),
        "gfd_poller_init_copy_engine": ([vp], c_int),
        "gfd_poller_init_direct_ce": ([vp], c_int),
        "gfd_poller_submit_direct": ([vp, vp, c_int], c_dbl),
        "gfd_poller_set_tiled_queue": ([vp, vp], None),
        "gfd_poller_set_sg_task_queue": ([vp, vp], c_int),
        "gfd_poller_start": ([vp], c_int),
        "gfd_poller_stop": ([vp], None),
        "gfd_poller_is_running": ([vp], c_int),
        "gfd_poller_get_stats": ([vp, ctypes.POINTER(PollerStats)], c_int),
        "gfd_poller_reset_stats": ([vp], None),
        "gfd_poller_get_info": ([vp, ctypes.POINTER(PollerInfo)], c_int),
        "gfd_poller_set_trace": ([vp, c_int], None),
        "gfd_poller_read_trace": ([vp, vp, c_int], c_int),
        "gfd_poller_set_copy_timing": ([vp, c_int], None),
        "gfd_poller_read_copy_times": ([vp, vp, c_int], c_int),
        "gfd_poller_copy_clock_ns": ([vp], c_u64),
        "gfd_poller_set_direct_chunk_bytes": ([vp, c_u64], None),
        "gfd_poller_set_direct_zero_copy_max_bytes": ([vp, c_u64], None),
        "gfd_poller_set_direct_zero_copy_min_bytes": ([vp, c_u64], c_u64),
        "gfd_poller_set_direct_zero_copy_head_bytes": ([vp, c_u64], c_u64),
        "gfd_poller_set_zero_copy_worker": ([vp, c_int], c_int),
        "gfd_poller_zero_copy_worker_stats": ([vp, ctypes.POINTER(c_u64), ctypes.POINTER(c_u64)], c_int),
        "gfd_poller_set_worker_queue_max_bytes": ([vp, c_u64], c_u64),
        "gfd_poller_zero_copy_worker_timeline": ([vp, vp, c_int], c_int),
        "gfd_bench_zero_copy_tokens_signal": ([vp, vp, c_u32, c_int, c_int, c_int, pd], c_int),
        "gfd_zero_copy_gather_tokens_signal": ([vp, vp, c_u32, c_int, vp, vp, c_u64, vp], c_int),
        "gfd_zero_copy_scatter_tokens_signal": ([vp, vp, c_u32, c_int, vp, vp, c_u64, vp], c_int),
        "gfd_zero_copy_gather_signal": ([vp, c_int, vp, vp, c_u64, vp], c_int),
        "gfd_zero_copy_gather_signal_presliced": ([vp, c_int, vp, vp, c_u64, vp], c_int),
        "gfd_zero_copy_target_waves": ([], c_int),
        "gfd_poller_set_gather_slice_bytes": ([vp, c_u64], None),
        "gfd_host_gather": ([vp, c_int, vp, c_u64, c_u64, c_int, vp, c_int], c_int),
        "gfd_staging_pool_init": ([c_int, c_sz, c_int], c_int),
        "gfd_staging_pool_shutdown": ([], None),
        "gfd_zero_copy_gather_tokens": ([vp, vp, c_u32, c_int, vp], c_int),
        "gfd_zero_copy_gather": ([vp, c_int, vp], c_int),
        "gfd_moe_route": ([vp, c_int, c_int, vp, vp, vp, vp], c_int),
        "gfd_moe_route_noalloc": ([vp, c_int, c_int, vp, vp, vp], c_int),
        "gfd_sg_gather_rmsnorm": ([vp, c_u64, c_int, vp, c_int, c_u32, vp, vp, vp, ctypes.c_float, c_int, vp, vp],
                                  c_int),
        "gfd_queue_alloc": ([pvp], c_int),
        "gfd_queue_free": ([vp], c_int),
        "gfd_queue_submit_tokens": ([vp, vp, vp, c_int, c_u32, c_u64, vp], c_int),
        "gfd_queue_wait": ([vp, c_u64, c_u64, vp, vp], c_int),
        "gfd_queue_submit_tokens_safe": ([vp, vp, vp, c_int, c_u32, c_u64, c_u64, vp, vp, vp], c_int),
        "gfd_bench_memcpy_per_token": ([vp, vp, c_int, c_u32, c_int, c_int, pd], c_int),
        "gfd_bench_memcpy_contiguous": ([vp, vp, c_sz, c_int, c_int, c_int, pd], c_int),
        "gfd_bench_sdma_contiguous": ([vp, vp, c_sz, c_int, c_int, c_int, c_int, pd, ctypes.POINTER(c_u32)], c_int),
        "gfd_bench_submit_direct": ([vp, vp, c_int, c_int, c_int, pd], c_int),
        "gfd_bench_host_gather": ([vp, c_int, c_int, vp, c_u64, c_int, vp, c_int, c_int, pd], c_int),
        "gfd_bench_zero_copy_tokens": ([vp, vp, c_u32, c_int, c_int, c_int, pd, pd], c_int),
        "gfd_zero_copy_scatter_tokens": ([vp, vp, c_u32, c_int, vp], c_int),
        "gfd_plan_expert_entries": ([vp, c_int, c_int, vp, c_u64, vp, c_u32, vp, vp, vp], c_int),
        "gfd_queue_fused_checksums": ([vp, vp, vp, c_int, c_u32, c_u64, c_u64, vp, vp, vp], c_int),
        "gfd_tiled_queue_alloc": ([pvp, c_u32, c_u32, c_u32, c_u32, c_int], c_int),
        "gfd_tiled_queue_free": ([vp], c_int),
        "gfd_tiled_queue_reset": ([vp], c_int),
        "gfd_tiled_poller_run": ([vp, vp, vp, c_int, c_u64, vp, vp, vp], c_int),
        "gfd_sg_task_queue_alloc": ([pvp, c_int], c_int),
        "gfd_sg_task_queue_free": ([vp], c_int),
        "gfd_sg_task_queue_reset": ([vp], c_int),
        "gfd_sg_poller_run": ([vp, vp, vp, vp, c_int, c_u32, c_u64, vp, vp, vp], c_int),
        "gfd_bench_zero_copy_scatter_tokens": ([vp, vp, c_u32, c_int, c_int, c_int, pd, pd], c_int),
        "gfd_bench_memcpy_contiguous_d2h": ([vp, vp, ctypes.c_size_t, c_int, c_int, c_int, pd], c_int),
        "gfd_bench_queue": ([vp, vp, vp, c_int, c_u32, ctypes.POINTER(c_u64), c_int, c_int, c_u64, pd], c_int),
        "gfd_warp_spec_run": ([vp, vp, c_u32, c_u32, c_u32, c_u32, c_int, c_int, c_int, c_int, vp, c_int, pd,
                               ctypes.POINTER(SessionResult)], c_int),
        "gfd_warp_spec_run_rms_sin": ([vp, vp, c_u32, c_u32, c_u32, c_u32, c_int, c_int, c_int, vp, c_int, pd,
                                       ctypes.POINTER(SessionResult)], c_int),
        "gfd_sg_session_create": ([c_int, c_int, c_u32, c_int, pvp], c_int),
        "gfd_sg_session_destroy": ([vp], None),
        "gfd_sg_session_submit": ([vp, vp, c_u32, c_u32, c_u32], ctypes.c_int64),
        "gfd_sg_session_launch": ([vp, vp, vp], c_int),
        "gfd_sg_session_launch_l2norm": ([vp, vp, c_u32, vp], c_int),
        "gfd_sg_session_launch_gpu_submit": ([vp, vp, c_u32, c_u32, vp, vp], c_int),
        "gfd_sg_session_synchronize": ([vp, c_u64], c_int),
        "gfd_sg_session_launch_moe": ([vp, vp, c_u64, c_int, vp, vp, c_int, c_int, c_u32, c_u32, vp, vp, vp,
                                       ctypes.c_float, vp], c_int),
        "gfd_sg_session_reset": ([vp], c_int),
        "gfd_sg_session_stats": ([vp, ctypes.POINTER(SessionResult)], c_int),
        "gfd_sg_session_queue": ([vp], vp),
        "gfd_sg_session_enable_trace": ([vp, c_u32], c_int),
        "gfd_sg_session_read_trace": ([vp, vp, c_u32, vp, c_u32, ctypes.POINTER(c_u32), ctypes.POINTER(c_u32)],
                                      c_int),
        "gfd_bench_sg_session": ([vp, vp, c_u32, c_u32, c_int, c_int, pd], c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    return sig


def lib():
    """Load libgfd_amd.so (ImportError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("libgfd_amd.so is not built (run: python -m gfd_amd.builder)")
        L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        _SIGNATURES.update(_declare(L))
        _lib = L
    return _lib


def bound_symbols():
    """Names of every C-ABI function this package binds."""
    return sorted(_SIGNATURES)


def _check(rc, what):
    if rc != 0:
        msg = lib().gfd_last_error().decode(errors="replace")
        raise GfdError("%s failed (%d): %s" % (what, rc, msg))


# ------------------------------------------------------------------ memory

class HostBuffer:
    """Pinned host memory (hipHostMalloc) with a numpy uint8 view."""

    def __init__(self, nbytes, flags=HOST_DEFAULT):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _check(lib().gfd_host_alloc(ctypes.byref(p), max(self.nbytes, 1), flags), "gfd_host_alloc")
        self.ptr = p.value
        self.array = np.ctypeslib.as_array((ctypes.c_uint8 * max(self.nbytes, 1)).from_address(self.ptr))[:self.nbytes]

    def free(self):
        if self.ptr:
            self.array = None
            lib().gfd_host_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceBuffer:
    """HBM allocation (hipMalloc)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _check(lib().gfd_device_alloc(ctypes.byref(p), max(self.nbytes, 1)), "gfd_device_alloc")
        self.ptr = p.value

    def fill(self, value):
        _check(lib().gfd_memset_device(self.ptr, value, self.nbytes), "gfd_memset_device")

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        _check(lib().gfd_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes), "gfd_memcpy_h2d")

    def download(self, nbytes=None, offset=0):
        n = self.nbytes - offset if nbytes is None else int(nbytes)
        out = np.empty(n, dtype=np.uint8)
        _check(lib().gfd_memcpy_d2h(out.ctypes.data, self.ptr + offset, n), "gfd_memcpy_d2h")
        return out

    def free(self):
        if self.ptr:
            lib().gfd_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    _check(lib().gfd_device_synchronize(), "gfd_device_synchronize")


def device_count():
    n = ctypes.c_int(0)
    rc = lib().gfd_device_count(ctypes.byref(n))
    return n.value if rc == 0 else 0


def make_entries(src_addrs, dst_base, token_size):
    """SGEntry array: entry j = {dst_base + j*token_size, src_addrs[j], token_size}."""
    src_addrs = np.asarray(src_addrs, dtype=np.uint64)
    n = len(src_addrs)
    arr = (SGEntry * max(n, 1))()
    a = np.frombuffer(arr, dtype=np.uint64).reshape(-1, 3)[:n]
    a[:, 0] = np.uint64(dst_base) + np.arange(n, dtype=np.uint64) * np.uint64(token_size)
    a[:, 1] = src_addrs
    a[:, 2] = token_size
    return arr


# ------------------------------------------------------------ host classes

class StagingPool:
    """gfd::StagingPool::instance() (reference include/gfd/staging_pool.h)."""

    @staticmethod
    def init(num_gpus, buf_size, numa_node=0):
        return lib().gfd_staging_pool_init(num_gpus, buf_size, numa_node) == 0

    @staticmethod
    def shutdown():
        lib().gfd_staging_pool_shutdown()


class CpuPollingThread:
    """gfd::CpuPollingThread (reference include/gfd/cpu_polling.h:19-84)."""

    def __init__(self, queue=None, gpu_base=None, cpu_base=None, total_cpu_size=0, use_ce=True, numa_node=0,
                 core_offset=0, num_ce_channels=0, exclusive_core_base=-1, exclusive_core_count=0):
        q = getattr(queue, "ptr", queue)
        self._h = lib().gfd_poller_create(q, gpu_base, cpu_base, total_cpu_size, int(bool(use_ce)), numa_node,
                                          core_offset, num_ce_channels, exclusive_core_base,
                                          exclusive_core_count)
        if not self._h:
            raise GfdError("gfd_poller_create failed")

    def init_copy_engine(self):
        return lib().gfd_poller_init_copy_engine(self._h) == 0

    def init_direct_ce(self):
        return lib().gfd_poller_init_direct_ce(self._h) == 0

    def submit_direct(self, entries, count=None):
        if count is None:
            count = len(entries)
        return lib().gfd_poller_submit_direct(self._h, ctypes.cast(entries, ctypes.c_void_p), count)

    def set_tiled_queue(self, tq):
        lib().gfd_poller_set_tiled_queue(self._h, getattr(tq, "ptr", tq))

    def set_sg_task_queue(self, sq):
        """Switched off: CpuPollingThread::start() refuses an SG task queue (an
        SG-mode run aborted the process on MI355X and the cause is not found).
        The C-ABI records the queue and reports GFD_ERR_NOT_SUPPORTED."""
        rc = lib().gfd_poller_set_sg_task_queue(self._h, getattr(sq, "ptr", sq))
        if rc != 0:
            raise RuntimeError(lib().gfd_last_error().decode())

    def start(self):
        """Start the polling thread; raises GfdError if it did not start."""
        _check(lib().gfd_poller_start(self._h), "CpuPollingThread.start")

    def is_running(self):
        return bool(lib().gfd_poller_is_running(self._h))

    def stop(self):
        lib().gfd_poller_stop(self._h)

    def stats(self):
        s = PollerStats()
        lib().gfd_poller_get_stats(self._h, ctypes.byref(s))
        return {k: getattr(s, k) for k, _ in PollerStats._fields_}

    def reset_stats(self):
        lib().gfd_poller_reset_stats(self._h)

    def info(self):
        i = PollerInfo()
        lib().gfd_poller_get_info(self._h, ctypes.byref(i))
        d = {k: getattr(i, k) for k, _ in PollerInfo._fields_}
        d["worker_cpus"] = list(i.worker_cpus)[: i.num_gather_workers]
        return d

    def set_trace(self, on=True):
        lib().gfd_poller_set_trace(self._h, int(bool(on)))

    def read_trace(self, max_events=16384):
        """Drain the timeline trace: structured array (t_ns, kind, a, b)."""
        buf = np.zeros(max_events, dtype=TRACE_DTYPE)
        n = lib().gfd_poller_read_trace(self._h, buf.ctypes.data, max_events)
        return buf[:n]

    def set_copy_timing(self, on=True):
        """Record engine start/end timestamps of every SDMA copy."""
        lib().gfd_poller_set_copy_timing(self._h, int(bool(on)))

    def read_copy_times(self, max_copies=65536):
        """Drain the copy timeline: structured array (seq, bytes, start_ns, end_ns, channel, engine, path)."""
        buf = np.zeros(max_copies, dtype=COPY_TIME_DTYPE)
        n = lib().gfd_poller_read_copy_times(self._h, buf.ctypes.data, max_copies)
        return buf[:n]

    def copy_clock_ns(self):
        return int(lib().gfd_poller_copy_clock_ns(self._h))

    def set_direct_chunk_bytes(self, b):
        lib().gfd_poller_set_direct_chunk_bytes(self._h, b)

    def set_direct_zero_copy_max_bytes(self, b):
        """Lists up to b bytes (destination-contiguous, pinned sources) use the
        zero-copy kernel; 0 = always the staged SDMA route."""
        lib().gfd_poller_set_direct_zero_copy_max_bytes(self._h, b)

    def set_direct_zero_copy_min_bytes(self, b):
        """Lists of at most b bytes take the staged SDMA route (default
        64 KiB).  Returns the previous value."""
        return int(lib().gfd_poller_set_direct_zero_copy_min_bytes(self._h, b))

    def set_zero_copy_worker(self, on=True):
        """The persistent zero-copy worker (CpuPollingThread::set_zero_copy_worker):
        Direct lists up to the zero-copy limit and Queue batches up to
        set_worker_queue_max_bytes() with pinned sources go through it."""
        _check(lib().gfd_poller_set_zero_copy_worker(self._h, int(bool(on))), "gfd_poller_set_zero_copy_worker")

    def zero_copy_worker_stats(self):
        """{"jobs": ..., "launches": ...} of the worker (0 while it is off)."""
        j, l = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().gfd_poller_zero_copy_worker_stats(self._h, ctypes.byref(j), ctypes.byref(l)),
               "gfd_poller_zero_copy_worker_stats")
        return {"jobs": j.value, "launches": l.value}

    def zero_copy_worker_timeline(self, max_jobs=64):
        """The worker's device timeline of its latest jobs, newest first: an
        (n, 8) uint64 array on the GPU's 100 MHz wall clock (the last
        workgroup to find the job, the last to hold it and its records,
        unused, the last done copying, unused, the last progress word stored,
        the job number, unused).  Empty unless GFD_ZC_WORKER_TRACE=1 was set
        when the worker started."""
        out = np.zeros((max_jobs, 8), np.uint64)
        n = lib().gfd_poller_zero_copy_worker_timeline(self._h, out.ctypes.data, max_jobs)
        return out[:n]

    def set_worker_queue_max_bytes(self, b):
        """Queue batches of at most b bytes go to the worker; returns the previous limit."""
        return int(lib().gfd_poller_set_worker_queue_max_bytes(self._h, b))

    def set_direct_zero_copy_head_bytes(self, b):
        """Larger lists (destination-contiguous, pinned sources): the zero-copy
        kernel moves the first entries, up to b bytes, while the rest is staged
        for the copy engines; 0 = staged only.  Returns the previous value."""
        return int(lib().gfd_poller_set_direct_zero_copy_head_bytes(self._h, b))

    def set_gather_slice_bytes(self, b):
        lib().gfd_poller_set_gather_slice_bytes(self._h, b)

    def close(self):
        if self._h:
            lib().gfd_poller_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TiledQueue:
    """gfd::TiledQueue (reference include/gfd/tiled_queue.h:8-43) in
    fine-grained host memory; ``ptr`` also serves as its DescriptorQueue."""

    def __init__(self, total_tiles, tokens_per_tile, tokens_per_chunk, token_size, device_signals=True):
        p = ctypes.c_void_p()
        _check(lib().gfd_tiled_queue_alloc(ctypes.byref(p), total_tiles, tokens_per_tile, tokens_per_chunk,
                                           token_size, int(bool(device_signals))), "gfd_tiled_queue_alloc")
        self.ptr = p.value
        self.total_tiles = total_tiles
        # TiledQueue: base (QUEUE_SIZE descriptors + 3 indices, 64-aligned),
        # TileScheduler (64 B), tile_chunk_done[MAX_TILES], d_tile_chunk_done.
        base_bytes = (QUEUE_SIZE * 64 + 3 * 8 + 63) // 64 * 64
        self._idx = np.ctypeslib.as_array((ctypes.c_uint64 * 3).from_address(self.ptr + QUEUE_SIZE * 64))
        self._done = np.ctypeslib.as_array((ctypes.c_uint64 * MAX_TILES).from_address(self.ptr + base_bytes + 64))
        self._dptr = (ctypes.c_uint64 * 1).from_address(self.ptr + base_bytes + 64 + MAX_TILES * 8)

    def reset(self):
        _check(lib().gfd_tiled_queue_reset(self.ptr), "gfd_tiled_queue_reset")

    @property
    def done_idx(self):
        return int(self._idx[2])

    def tile_progress(self):
        """Per-tile cumulative landed-token counts (HBM words when allocated there)."""
        n = self.total_tiles
        if self._dptr[0]:
            out = np.zeros(n, np.uint64)
            _check(lib().gfd_memcpy_d2h(out.ctypes.data, self._dptr[0], n * 8), "gfd_memcpy_d2h")
            return out
        return self._done[:n].copy()

    def free(self):
        if self.ptr:
            self._idx = self._done = self._dptr = None
            lib().gfd_tiled_queue_free(self.ptr)
            self.ptr = None


def tiled_poller_run(tq, cpu_base, gpu_base, sums_ptr, status_ptr, whole_tile=False, timeout_us=10_000_000,
                     stream=None):
    """Kernel-driven tiled mode (see gfd_tiled_poller_run in include/gfd_capi.h)."""
    _check(lib().gfd_tiled_poller_run(tq.ptr, cpu_base, gpu_base, int(bool(whole_tile)), timeout_us, sums_ptr,
                                      status_ptr, stream), "gfd_tiled_poller_run")


class SGTaskQueue:
    """gfd::SGTaskQueue for the poller's SG mode (set_sg_task_queue), with its
    d_list_done flags in HBM (device_flags) or fine-grained host memory."""

    def __init__(self, device_flags=True):
        p = ctypes.c_void_p()
        _check(lib().gfd_sg_task_queue_alloc(ctypes.byref(p), int(bool(device_flags))), "gfd_sg_task_queue_alloc")
        self.ptr = p.value
        self.device_flags = bool(device_flags)

    # Field offsets in gfd::SGTaskQueue (static_asserts in sg_poller_kernels.hip).
    _LISTS_COMPLETED = 409856
    _D_LIST_DONE = 409872

    def reset(self):
        _check(lib().gfd_sg_task_queue_reset(self.ptr), "gfd_sg_task_queue_reset")

    @property
    def lists_completed(self):
        return int(ctypes.c_uint64.from_address(self.ptr + self._LISTS_COMPLETED).value)

    def list_done(self, n):
        """d_list_done[0:n] (read from HBM or host memory, wherever it lives)."""
        p = int(ctypes.c_uint64.from_address(self.ptr + self._D_LIST_DONE).value)
        out = np.zeros(n, np.uint64)
        if self.device_flags:
            _check(lib().gfd_memcpy_d2h(out.ctypes.data, p, n * 8), "gfd_memcpy_d2h")
        else:
            out[:] = np.ctypeslib.as_array((ctypes.c_uint64 * n).from_address(p))
        return out

    def free(self):
        if self.ptr:
            lib().gfd_sg_task_queue_free(self.ptr)
            self.ptr = None


def sg_poller_run(queue, sg_queue, d_entries_ptr, d_offsets_ptr, num_lists, total_entries, sums_ptr, status_ptr,
                  timeout_us=10_000_000, stream=None):
    """Kernel-driven SG mode (see gfd_sg_poller_run in include/gfd_capi.h)."""
    _check(lib().gfd_sg_poller_run(queue.ptr, sg_queue.ptr, d_entries_ptr, d_offsets_ptr, num_lists, total_entries,
                                   timeout_us, sums_ptr, status_ptr, stream), "gfd_sg_poller_run")


class DescriptorQueue:
    """gfd::DescriptorQueue in fine-grained host memory."""

    def __init__(self):
        p = ctypes.c_void_p()
        _check(lib().gfd_queue_alloc(ctypes.byref(p)), "gfd_queue_alloc")
        self.ptr = p.value
        base = self.ptr + QUEUE_SIZE * 64
        self._idx = np.ctypeslib.as_array((ctypes.c_uint64 * 3).from_address(base))

    @property
    def write_idx(self):
        return int(self._idx[0])

    @property
    def read_idx(self):
        return int(self._idx[1])

    @property
    def done_idx(self):
        return int(self._idx[2])

    def free(self):
        if self.ptr:
            self._idx = None
            lib().gfd_queue_free(self.ptr)
            self.ptr = None


def host_gather(entries, count, out, chunk_bytes=0, slice_bytes=0, num_workers=0):
    """Run the product's gather engine on the host only; returns the chunk
    completion order (see gfd_host_gather in include/gfd_capi.h)."""
    out_ptr = out.ctypes.data if isinstance(out, np.ndarray) else out
    total = sum(int(entries[i].size) for i in range(count)) if count else 0
    # Every chunk but the last is at least min(64 KiB, chunk_bytes).
    cap = total // (min(65536, chunk_bytes) if chunk_bytes else 65536) + 2
    order = np.full(cap, -1, dtype=np.int32)
    n = lib().gfd_host_gather(ctypes.cast(entries, ctypes.c_void_p), count, out_ptr, chunk_bytes, slice_bytes,
                              num_workers, order.ctypes.data, cap)
    if n < 0:
        _check(-1, "gfd_host_gather")
    if n > cap:
        raise GfdError("gfd_host_gather reported %d chunks, more than the %d it may" % (n, cap))
    return order[:n]


def zero_copy_gather_tokens(src_addrs_ptr, dst_ptr, token_size, num_tokens, stream=None):
    _check(lib().gfd_zero_copy_gather_tokens(src_addrs_ptr, dst_ptr, token_size, num_tokens, stream),
           "gfd_zero_copy_gather_tokens")


def plan_expert_entries(routing_ptr, num_tokens, expert, cpu_base, stride, gpu_dst, token_size, entries_ptr,
                        count_ptr, stream=None):
    """GPU-built SG list (examples/03_gpu_planned_transfer.cu): the tokens
    routed to `expert`, in token order, as gfd_sg_entry records written to
    entries_ptr (pinned host or HBM); the match count goes to count_ptr."""
    _check(lib().gfd_plan_expert_entries(routing_ptr, num_tokens, expert, cpu_base, stride, gpu_dst, token_size,
                                         entries_ptr, count_ptr, stream), "gfd_plan_expert_entries")


def zero_copy_scatter_tokens(dst_addrs_ptr, src_ptr, token_size, num_tokens, stream=None):
    """Offload (reverse path): dst_addrs[j] (pinned host) <- src + j*token_size (HBM)."""
    _check(lib().gfd_zero_copy_scatter_tokens(dst_addrs_ptr, src_ptr, token_size, num_tokens, stream),
           "gfd_zero_copy_scatter_tokens")


def zero_copy_gather(entries_ptr, count, stream=None):
    _check(lib().gfd_zero_copy_gather(entries_ptr, count, stream), "gfd_zero_copy_gather")


def moe_route(d_logits, num_tokens, num_experts, d_top2, d_offsets, d_row_token, stream=None):
    _check(lib().gfd_moe_route(d_logits, num_tokens, num_experts, d_top2, d_offsets, d_row_token, stream),
           "gfd_moe_route")


def sg_gather_rmsnorm(host_base, token_stride, num_tokens, d_row_token, num_rows, row_bytes, d_dst, d_out=None,
                      d_weight=None, eps=1e-6, num_blocks=0, d_error=None, stream=None):
    _check(lib().gfd_sg_gather_rmsnorm(host_base, token_stride, num_tokens, d_row_token, num_rows, row_bytes, d_dst,
                                       d_out, d_weight, eps, num_blocks, d_error, stream), "gfd_sg_gather_rmsnorm")


def warp_spec_run(cpu_src, gpu_dst, total_tokens, token_size, tokens_per_tile=128, tokens_per_chunk=0,
                  double_buffer=False, per_tile_mode=False, num_blocks=0, token_sums=None, iters=1,
                  helper_waves=-1):
    """WarpSpecSession (reference include/gfd/warp_spec_session.h:14-132) over
    tokens [0, total_tokens): construct, then `iters` times launch +
    synchronize.  token_sums: device float[total_tokens] for the per-token
    sum consumer, or None for a no-op consumer.  helper_waves: transfer
    helper waves per workgroup (negative: about 32 transfer waves per launch,
    at most 3 helpers; fewer if the workgroup would pass 1024 threads).
    Returns (result dict, kernel times in ms)."""
    res = SessionResult()
    times = np.zeros(max(iters, 1), dtype=np.float64)
    _check(lib().gfd_warp_spec_run(cpu_src, gpu_dst, total_tokens, token_size, tokens_per_tile, tokens_per_chunk,
                                   int(bool(double_buffer)), int(bool(per_tile_mode)), num_blocks, helper_waves,
                                   token_sums, iters,
                                   times.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), ctypes.byref(res)),
           "gfd_warp_spec_run")
    return res.as_dict(), times


def warp_spec_run_rms_sin(cpu_src, gpu_dst, total_tokens, token_size, out, tokens_per_tile=128,
                          tokens_per_chunk=0, double_buffer=False, num_blocks=0, iters=1, helper_waves=-1):
    """warp_spec_run with the RMSNorm + sinf consumer of the reference's
    examples/07_warp_spec_simple.cu (out: device float[total_tokens], token t
    -> sum of sin(x r) x r over its floats, r = 1/sqrt(mean(x^2) + 1e-6)).
    Returns (result dict, kernel times in ms)."""
    res = SessionResult()
    times = np.zeros(max(iters, 1), dtype=np.float64)
    _check(lib().gfd_warp_spec_run_rms_sin(cpu_src, gpu_dst, total_tokens, token_size, tokens_per_tile,
                                           tokens_per_chunk, int(bool(double_buffer)), num_blocks, helper_waves, out,
                                           iters, times.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                                           ctypes.byref(res)), "gfd_warp_spec_run_rms_sin")
    return res.as_dict(), times


def device_sg_entries(src, dst, size, tag=0):
    """Structured array of DeviceSGEntry rows (numpy, 24 bytes each)."""
    src = np.asarray(src, dtype=np.uint64)
    a = np.zeros(len(src), dtype=DEVICE_SG_ENTRY_DTYPE)
    a["src"] = src
    a["dst"] = np.asarray(dst, dtype=np.uint64)
    a["size"] = size
    a["tag"] = tag
    return a


# gfd_sg_trace_list / gfd_sg_trace_block (include/gfd_capi.h).
SG_TRACE_LIST_DTYPE = np.dtype([("claimed", "<u8"), ("ready", "<u8"), ("landed", "<u8"), ("block", "<u4"),
                                ("list_id", "<u4")])
SG_TRACE_BLOCK_DTYPE = np.dtype([("start", "<u8"), ("exit", "<u8"), ("lists", "<u8"), ("hw", "<u8")])
SG_TRACE_TICKS_PER_US = 100  # the device wall clock runs at 100 MHz


class SGWarpSpecSession:
    """gfd::SGWarpSpecSession (reference include/gfd/warp_spec_session.h:142-258,
    src/sg_warp_spec_session.cpp) with the built-in consumers of the C-ABI."""

    def __init__(self, num_compute_warps=1, num_blocks=0, idle_limit_ms=0, helper_waves=-1):
        """helper_waves: transfer helper waves per workgroup, 0..3 (negative:
        about 32 transfer waves per launch, at most 3 helpers)."""
        h = ctypes.c_void_p()
        _check(lib().gfd_sg_session_create(num_compute_warps, num_blocks, idle_limit_ms, helper_waves,
                                           ctypes.byref(h)),
               "gfd_sg_session_create")
        self._h = h.value

    def submit_sg_list(self, entries, list_id, flags=SG_FLAG_HOST_SUBMITTED):
        """entries: DEVICE_SG_ENTRY_DTYPE array.  Returns the ring index."""
        entries = np.ascontiguousarray(entries, dtype=DEVICE_SG_ENTRY_DTYPE)
        idx = lib().gfd_sg_session_submit(self._h, entries.ctypes.data if len(entries) else None, len(entries),
                                          list_id, flags)
        if idx < 0:
            _check(1, "gfd_sg_session_submit")
        return idx

    def launch(self, list_sums=None, stream=None):
        _check(lib().gfd_sg_session_launch(self._h, list_sums, stream), "gfd_sg_session_launch")

    def launch_l2norm(self, out, out_len, stream=None):
        """Launch with the per-entry fp32 L2-norm consumer (out: device float[out_len])."""
        _check(lib().gfd_sg_session_launch_l2norm(self._h, out, out_len, stream), "gfd_sg_session_launch_l2norm")

    def launch_gpu_submit(self, d_entries, entries_per_list, num_lists, list_sums=None, stream=None):
        _check(lib().gfd_sg_session_launch_gpu_submit(self._h, d_entries, entries_per_list, num_lists, list_sums,
                                                      stream), "gfd_sg_session_launch_gpu_submit")

    def launch_moe(self, host_base, token_stride, num_tokens, d_offsets, d_row_token, num_experts, num_rows,
                   row_bytes, d_dst, d_out=None, d_weight=None, eps=1e-6, rows_per_list=48, stream=None):
        """The MoE-routed gather with GPU-built lists (gfd_sg_session_launch_moe);
        the kernel ends itself once every list has landed."""
        _check(lib().gfd_sg_session_launch_moe(self._h, host_base, token_stride, num_tokens, d_offsets, d_row_token,
                                               num_experts, num_rows, row_bytes, rows_per_list, d_dst, d_out,
                                               d_weight, eps, stream), "SGWarpSpecSession.launch_moe")

    def synchronize(self, extra_gpu_lists=0):
        _check(lib().gfd_sg_session_synchronize(self._h, extra_gpu_lists), "gfd_sg_session_synchronize")

    def reset(self):
        _check(lib().gfd_sg_session_reset(self._h), "gfd_sg_session_reset")

    def stats(self):
        r = SessionResult()
        _check(lib().gfd_sg_session_stats(self._h, ctypes.byref(r)), "gfd_sg_session_stats")
        return r.as_dict()

    def queue_ptr(self):
        return lib().gfd_sg_session_queue(self._h)

    def enable_trace(self, max_lists):
        """Record the first max_lists lists and every workgroup of each later
        launch (0 switches it off); read them with trace() after synchronize()."""
        _check(lib().gfd_sg_session_enable_trace(self._h, max_lists), "gfd_sg_session_enable_trace")
        self._trace_cap = max_lists

    def trace(self):
        """The last launch's timeline: (lists, blocks) structured arrays
        (SG_TRACE_LIST_DTYPE in ring order, SG_TRACE_BLOCK_DTYPE per
        workgroup), in ticks of the device's 100 MHz wall clock."""
        cap = getattr(self, "_trace_cap", 0)
        nb = self.stats()["grid"]
        lists = np.zeros(cap, dtype=SG_TRACE_LIST_DTYPE)
        blocks = np.zeros(nb, dtype=SG_TRACE_BLOCK_DTYPE)
        n_l, n_b = ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib().gfd_sg_session_read_trace(self._h, lists.ctypes.data if cap else None, cap,
                                               blocks.ctypes.data if nb else None, nb, ctypes.byref(n_l),
                                               ctypes.byref(n_b)), "gfd_sg_session_read_trace")
        return lists[:n_l.value], blocks[:n_b.value]

    def bench(self, entries, entries_per_list, warmup=2, iters=10):
        entries = np.ascontiguousarray(entries, dtype=DEVICE_SG_ENTRY_DTYPE)
        t = np.zeros(iters, dtype=np.float64)
        _check(lib().gfd_bench_sg_session(self._h, entries.ctypes.data, len(entries), entries_per_list, warmup, iters,
                                          t.ctypes.data_as(ctypes.POINTER(ctypes.c_double))), "gfd_bench_sg_session")
        return t

    def close(self):
        if self._h:
            lib().gfd_sg_session_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


SgWarpSpecSession = SGWarpSpecSession


def build(verbose=False):
    """Compile libgfd_amd.so for gfx950 (see gfd_amd/builder.py)."""
    from . import builder

    return builder.build(verbose=verbose)
