"""Python mirror of the native backend interface (names follow LeanStream's
backends/triton/binding.py ``NativeBackend`` and backends/triton/mapped.py ``Mapped``).

Device memory and streams come from PyTorch; every computation runs in the HIP
library through its C ABI. Errors from the library raise RuntimeError.
"""
import ctypes as C
import time

import numpy as np

from . import _native
from ._native import DeviceQueue, Epilogue, ExecDesc, LayerBuffers

MODE_BATCH_COMPAT, MODE_PROGRESSIVE, MODE_AUTO = 0, 1, 2
STATUS_TIMEOUT, STATUS_QUEUE_ERROR, STATUS_BAD_DESCRIPTOR, STATUS_RANGE, STATUS_QUEUE_UNCONSUMED = 1, 2, 4, 8, 16
EBUSY = 16
STAGE_ARM = C.CFUNCTYPE(C.c_int, C.c_void_p)   # int (*arm_final_prediction)(void*)
QUEUE_CONTROL_BYTES = 128


def _ptr(obj):
    if obj is None:
        return None
    if isinstance(obj, int):
        return obj
    if hasattr(obj, "data_ptr"):
        return obj.data_ptr()
    if isinstance(obj, Mapped):
        return obj.ptr
    raise TypeError(f"cannot take a device address of {type(obj)}")


class Mapped:
    """Fine-grained coherent host memory visible to the GPU at system scope
    (mapped.py:6-18: tm_alloc / tm_release / tm_acquire_all)."""

    def __init__(self, count, dtype):
        self.lib = _native.library()
        self.dtype = np.dtype(dtype)
        self.count = int(count)
        self.nbytes = max(1, self.count * self.dtype.itemsize)
        self.ptr = self.lib.ls_hip_host_alloc(self.nbytes)
        if not self.ptr:
            raise MemoryError("coherent host allocation failed")
        raw = (C.c_uint8 * self.nbytes).from_address(self.ptr)
        self.host = np.ctypeslib.as_array(raw).view(self.dtype)[: self.count]

    def release(self, index, value):
        self.lib.ls_hip_release_u32(self.ptr, int(index), int(value))

    def wait(self, value, count=None, timeout_ms=5000):
        n = self.count if count is None else count
        if self.lib.ls_hip_acquire_all(self.ptr, n, int(value), timeout_ms):
            raise RuntimeError("Mapped acquire timeout")

    def close(self):
        if self.ptr:
            self.host = None
            self.lib.ls_hip_host_free(self.ptr)
            self.ptr = None


class ReadyQueue:
    """DeviceExecQueue storage in coherent host memory plus the native
    ExecutionQueue producer (execution_queue.h:13-34)."""

    def __init__(self, capacity):
        self.lib = _native.library()
        self.capacity = int(capacity)
        self.descriptors = Mapped(max(1, self.capacity) * 5, np.uint32)
        self.indices = Mapped(max(1, self.capacity), np.uint32)
        self.control = Mapped(QUEUE_CONTROL_BYTES // 4, np.uint32)
        self.view = DeviceQueue(self.descriptors.ptr, self.indices.ptr, self.control.ptr, self.capacity)
        self.handle = self.lib.ls_queue_create(C.byref(self.view))
        if not self.handle:
            raise MemoryError("queue allocation failed")

    def write_descriptors(self, rows):
        rows = np.asarray(rows, dtype=np.uint32).reshape(-1, 5)
        if len(rows) > self.capacity:
            raise ValueError("more descriptors than queue capacity")
        self.descriptors.host[: rows.size] = rows.reshape(-1)

    def reset(self, epoch):
        self.lib.ls_queue_reset(self.handle, epoch)

    def prepare(self, total):
        self.lib.ls_queue_prepare(self.handle, total)

    def append_unpublished(self, index):
        self.lib.ls_queue_append_unpublished(self.handle, index)

    def activate(self):
        self.lib.ls_queue_activate(self.handle)

    def seal(self, total):
        self.lib.ls_queue_seal(self.handle, total)

    def publish_all(self):
        self.lib.ls_queue_publish_all(self.handle)

    def publish(self, index):
        self.lib.ls_queue_publish(self.handle, index)

    def fail(self, error):
        self.lib.ls_queue_fail(self.handle, error)

    def words(self):
        """QueueControl as a dict of its named 32-bit words."""
        w = self.control.host
        return dict(ready_count=int(w[0]), total_count=int(w[2]), epoch=int(w[3]), batch_epoch=int(w[4]),
                    error=int(w[5]), consumer_path=int(w[6]), claim_count=int(w[16]))

    def start_publisher(self, order, offsets_ns, fail_after=None, fail_code=0):
        order = np.ascontiguousarray(order, dtype=np.uint32)
        offs = np.ascontiguousarray(offsets_ns, dtype=np.uint64)
        fail_after = len(order) + 1 if fail_after is None else int(fail_after)
        handle = self.lib.ls_publisher_start(self.handle, order.ctypes.data, offs.ctypes.data, len(order), fail_after,
                                             fail_code)
        if not handle:
            raise RuntimeError("publisher start failed")
        return Publisher(self.lib, handle)

    def close(self):
        if self.handle:
            self.lib.ls_queue_destroy(self.handle)
            self.handle = None
        for m in (self.descriptors, self.indices, self.control):
            m.close()


class Publisher:
    def __init__(self, lib, handle):
        self.lib, self.handle = lib, handle

    def join(self):
        if self.handle:
            self.lib.ls_publisher_join(self.handle)
            self.handle = None


class NativeBackend:
    """The HIP ComputeBackend. Keep every bound tensor alive until GPU completion."""

    def __init__(self, offline_table=None):
        self.lib = _native.library()
        self._table = None
        if offline_table is None:
            self.context = self.lib.ls_hip_create()
        else:
            layers, buckets = len(offline_table), len(offline_table[0])
            if not all(len(row) == buckets for row in offline_table):
                raise ValueError("Ragged LUT")
            self._table = (C.c_uint8 * (layers * buckets))(*(v for row in offline_table for v in row))
            self.context = self.lib.ls_hip_create_table(self._table, layers, buckets)
        if not self.context:
            raise MemoryError("Native backend allocation failed")
        self._bound = None

    def bind(self, width, group_size, slot_capacity, cache, scales, physical_groups, cache_groups, staging=None,
             staging_groups=0, queue_capacity=0, hidden=None, partial=None, y32=None, executions=None,
             first_compute=None, claim_log=None, batch=1, stamps=None):
        b = LayerBuffers(width, group_size, batch, slot_capacity, cache_groups, staging_groups, physical_groups,
                         queue_capacity, _ptr(cache), _ptr(staging), _ptr(scales), _ptr(hidden), _ptr(partial),
                         _ptr(y32), _ptr(executions), _ptr(first_compute), _ptr(claim_log), _ptr(stamps))
        rc = self.lib.ls_hip_bind(self.context, C.byref(b))
        if rc:
            raise RuntimeError(f"Native bind failed: {rc}")
        self._bound = (b, cache, scales, staging, hidden, partial, y32, executions, first_compute, claim_log, stamps)

    def set_epilogue(self, residual, hidden, hidden_flag=None, norm_weight=None, norm_output=None, norm_flag=None,
                     bell=None, eps=0.0):
        """Install the layer epilogue (ls_hip_set_epilogue); every argument None removes it."""
        if residual is None and hidden is None:
            rc = self.lib.ls_hip_set_epilogue(self.context, None)
        else:
            e = Epilogue(_ptr(residual), _ptr(hidden), _ptr(hidden_flag), _ptr(norm_weight), _ptr(norm_output),
                         _ptr(norm_flag), _ptr(bell), float(eps))
            rc = self.lib.ls_hip_set_epilogue(self.context, C.byref(e))
            self._epilogue = (e, residual, hidden, hidden_flag, norm_weight, norm_output, norm_flag, bell)
        if rc:
            raise RuntimeError(f"Native set_epilogue failed: {rc}")

    def set_stage_hook(self, arm=None, b_done=None):
        """ls_hip_set_stage_hook: `arm` (a Python callable returning an int, or None) runs at
        the consumer -> reduction boundary of every later enqueue; `b_done` is a hipEvent_t
        handle recorded there (or None)."""
        fn = STAGE_ARM(lambda _ctx: int(arm())) if arm is not None else None
        rc = self.lib.ls_hip_set_stage_hook(self.context, C.cast(fn, C.c_void_p) if fn else None, None, b_done)
        if rc:
            raise RuntimeError(f"Native set_stage_hook failed: {rc}")
        self._stage_hook = fn   # kept alive while the library may call it

    def enqueue(self, layer, io_bucket, epoch, x, y, stream, core, core_count, queue, mode=MODE_PROGRESSIVE):
        rc = self.lib.ls_hip_enqueue(self.context, layer, io_bucket, epoch, _ptr(x), _ptr(y), stream, _ptr(core),
                                     core_count, C.byref(queue.view), mode)
        if rc:
            raise RuntimeError(f"Native enqueue failed: {rc}")

    def try_enqueue(self, layer, io_bucket, epoch, x, y, stream, core, core_count, queue, mode=MODE_PROGRESSIVE):
        return self.lib.ls_hip_enqueue(self.context, layer, io_bucket, epoch, _ptr(x), _ptr(y), stream, _ptr(core),
                                       core_count, C.byref(queue.view), mode)

    @staticmethod
    def chain_blocks(layers):
        """ls_hip_chain_layer blocks (a ctypes array) from a list of dicts with the struct's
        field names (device tensors or integer addresses); reusable across enqueues."""
        arr = (_native.ChainLayer * len(layers))()
        for dst, src in zip(arr, layers):
            for name, kind in _native.ChainLayer._fields_:
                if name in src:
                    v = src[name]
                    setattr(dst, name, _ptr(v) if kind is _native.p else float(v) if kind is C.c_float else int(v))
        return arr

    def try_enqueue_chain(self, layers, stream):
        """ls_hip_enqueue_chain over `layers` (dicts, or blocks from chain_blocks); returns the
        library's code."""
        arr = layers if isinstance(layers, C.Array) else self.chain_blocks(layers)
        return self.lib.ls_hip_enqueue_chain(self.context, arr, len(arr), stream)

    def enqueue_chain(self, layers, stream, wait_busy=True):
        """As try_enqueue_chain, raising on failure. EBUSY (more records in flight than the
        ring holds) is waited out while earlier launches complete, unless wait_busy is False."""
        arr = layers if isinstance(layers, C.Array) else self.chain_blocks(layers)
        while True:
            rc = self.try_enqueue_chain(arr, stream)
            if rc != EBUSY or not wait_busy:
                break
            time.sleep(0)
        if rc:
            raise RuntimeError(f"Native enqueue_chain failed: {rc}")

    def set_chain_stamps(self, stamps, layers):
        rc = self.lib.ls_hip_set_chain_stamps(self.context, _ptr(stamps), layers)
        if rc:
            raise RuntimeError(f"Native set_chain_stamps failed: {rc}")
        self._chain_stamps = stamps

    @property
    def chain_workers(self):
        return int(self.lib.ls_hip_chain_workers(self.context))

    @property
    def last_seq(self):
        return int(self.lib.ls_hip_last_seq(self.context))

    @property
    def done_seq(self):
        return int(self.lib.ls_hip_done_seq(self.context))

    def complete(self, layer=0):
        return bool(self.lib.ls_hip_complete(self.context, layer))

    def status(self):
        return int(self.lib.ls_hip_status(self.context))

    def clear_status(self):
        self.lib.ls_hip_clear_status(self.context)

    def set_spin_limit(self, ticks):
        self.lib.ls_hip_set_spin_limit(self.context, int(ticks))

    def set_workers(self, workers=0):
        """Override the persistent worker count (0 = the selected candidate's)."""
        self.lib.ls_hip_set_workers(self.context, int(workers))

    @property
    def slices(self):
        return int(self.lib.ls_hip_slices(self.context))

    @property
    def max_workers(self):
        return int(self.lib.ls_hip_max_workers(self.context))

    def select(self, layer, bucket):
        return int(self.lib.ls_hip_select(self.context, layer, bucket))

    def last_candidate(self):
        return int(self.lib.ls_hip_last_candidate(self.context))

    def close(self):
        # Caller must prove GPU completion before dropping buffers.
        if self.context:
            self.lib.ls_hip_destroy(self.context)
            self.context = None


def rank_groups(scores, k):
    """Native top-k (score desc, id asc); raises on non-finite scores."""
    lib = _native.library()
    s = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.zeros(max(1, k), dtype=np.int32)
    rc = lib.ls_rank_groups(s.ctypes.data, len(s), k, out.ctypes.data)
    if rc:
        raise ValueError(f"rank_groups failed: {rc}")
    return out[:k].astype(np.int64)


def quantize_io_load(remaining, total, buckets=8):
    return int(_native.library().ls_quantize_io_load(remaining, total, buckets))
