"""The C ABI of libleanstream_hip.so on the CPU (no GPU calls): exported symbols, the
ready-queue producer on host memory, kernel selection, ranking."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import oracle
from leanstream_amd import _native
from leanstream_amd._native import DeviceQueue

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "leanstream_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ls_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_entry_point_is_exported_and_bound():
    lib = _native.library()
    names = declared_functions()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/leanstream_hip.h but not exported"
    assert sorted(_native.EXPORTED) == names, "ctypes signatures and the header disagree"


class HostQueue:
    """DeviceExecQueue over plain numpy memory (the producer never touches the GPU)."""

    def __init__(self, capacity):
        self.desc = np.zeros(capacity * 5, dtype=np.uint32)
        self.idx = np.zeros(capacity, dtype=np.uint32)
        self.ctrl = np.zeros(32, dtype=np.uint32)   # 128-byte QueueControl
        self.view = DeviceQueue(self.desc.ctypes.data, self.idx.ctypes.data, self.ctrl.ctypes.data, capacity)
        self.lib = _native.library()
        self.h = self.lib.ls_queue_create(C.byref(self.view))
        assert self.h

    def words(self):
        c = self.ctrl
        return dict(ready=int(c[0]), total=int(c[2]), epoch=int(c[3]), batch=int(c[4]), error=int(c[5]))

    def close(self):
        self.lib.ls_queue_destroy(self.h)


def test_queue_publication_order_and_first_error_wins():
    """execution_queue.cpp:4-46; open_source_runtime_test.cpp:61-67 (order {2,0,3,1})."""
    q = HostQueue(8)
    lib = q.lib
    lib.ls_queue_reset(q.h, 7)
    lib.ls_queue_seal(q.h, 4)
    assert q.words() == dict(ready=0, total=4, epoch=7, batch=0, error=0)
    for i in (2, 0, 3, 1):
        lib.ls_queue_publish(q.h, i)
    assert q.words() == dict(ready=4, total=4, epoch=7, batch=7, error=0)
    assert q.idx[:4].tolist() == [2, 0, 3, 1]
    lib.ls_queue_reset(q.h, 9)
    lib.ls_queue_prepare(q.h, 5)
    lib.ls_queue_append_unpublished(q.h, 3)
    lib.ls_queue_append_unpublished(q.h, 0)
    assert q.words()["epoch"] == 0          # nothing visible before activation
    lib.ls_queue_activate(q.h)
    assert q.words() == dict(ready=2, total=5, epoch=9, batch=0, error=0)
    lib.ls_queue_fail(q.h, 5)
    lib.ls_queue_fail(q.h, 7)
    assert q.words()["error"] == 5
    lib.ls_queue_reset(q.h, 10)
    lib.ls_queue_seal(q.h, 3)
    lib.ls_queue_publish_all(q.h)
    assert q.words() == dict(ready=3, total=3, epoch=10, batch=10, error=0)
    assert q.idx[:3].tolist() == [0, 1, 2]
    q.close()


def test_quantize_io_load_known_answers():
    """kernel_selector_test.cpp:20-26."""
    f = _native.library().ls_quantize_io_load
    big = 0xFFFFFFFF
    assert f(1, 1, 8) == 7 and f(10, 8, 8) == 7
    assert f(0, 0, 8) == 0 and f(1, 0, 8) == 0 and f(1, 8, 0) == 0 and f(0, 8, 8) == 0
    assert [f(i, 8, 8) for i in range(8)] == list(range(8))
    assert f(big - 1, big, 8) == 7 and f(big - 1, big, big) == big - 1


def test_hip_selector_table_and_fallback():
    """kernel_selector.cpp:4-22 over the CDNA4 catalog: valid ids are taken from the
    table, anything else (id out of the catalog, layer/bucket out of range) falls back
    to the default candidate."""
    lib = _native.library()
    table = (C.c_uint8 * 6)(0, 1, 2, 3, 4, 255)
    ctx = lib.ls_hip_create_table(table, 1, 6)
    assert ctx
    try:
        assert [lib.ls_hip_select(ctx, 0, b) for b in range(5)] == [0, 1, 2, 3, 4]
        default = lib.ls_hip_select(ctx, 0, 5)
        assert default == 5   # kHipDefault: the ready-pair candidate
        assert lib.ls_hip_select(ctx, 1, 0) == default and lib.ls_hip_select(ctx, 0, 6) == default
        assert lib.ls_hip_last_candidate(ctx) == -1      # nothing enqueued yet
    finally:
        lib.ls_hip_destroy(ctx)
    ctx = lib.ls_hip_create()
    assert lib.ls_hip_select(ctx, 3, 3) == 5
    lib.ls_hip_destroy(ctx)


def test_compute_backend_view_size_check():
    lib = _native.library()
    ctx = lib.ls_hip_create()
    buf = (C.c_uint8 * 64)()
    assert lib.ls_hip_compute_backend(ctx, buf, 8) != 0          # too small for the struct
    assert lib.ls_hip_compute_backend(ctx, buf, 64) == 0
    ptrs = np.frombuffer(bytes(buf), dtype=np.uint64)[:6]
    assert ptrs[0] == ctx and ptrs[1] != 0 and ptrs[2] != 0     # context, enqueue, complete
    lib.ls_hip_destroy(ctx)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_rank_groups_matches_oracle(seed):
    """predictor_cpu.cpp:192-201: top-k by (score desc, id asc)."""
    rng = np.random.default_rng(seed)
    scores = rng.standard_normal(448).astype(np.float32)
    scores[rng.integers(0, 448, 40)] = 0.5     # ties
    lib = _native.library()
    for k in (0, 1, 58, 90, 448):
        out = np.zeros(max(1, k), dtype=np.int32)
        assert lib.ls_rank_groups(scores.ctypes.data, len(scores), k, out.ctypes.data) == 0
        assert out[:k].tolist() == oracle.rank(scores, k).tolist()
    bad = scores.copy()
    bad[3] = np.nan
    out = np.zeros(4, dtype=np.int32)
    assert lib.ls_rank_groups(bad.ctypes.data, len(bad), 4, out.ctypes.data) != 0


def test_stream_create_rejects_invalid_setup():
    """ls_stream_create validates its setup before touching the GPU."""
    lib = _native.library()
    assert not lib.ls_stream_create(None)
    s = _native.StreamSetup()          # all zero: no backend, no store, no geometry
    assert not lib.ls_stream_create(C.byref(s))
    s = _native.StreamSetup(1, 1, 1, 1, 1, 1, 1, 8, 1, 33, 0, 1, 0, 1, 0)   # qd above 32
    assert not lib.ls_stream_create(C.byref(s))
    s = _native.StreamSetup(1, 1, 1, 1, 1, 1, 1, 8, 1, 8, 2, 1, 0, 1, 0)    # unknown copy engine
    assert not lib.ls_stream_create(C.byref(s))
    assert lib.ls_stream_run(None, None, 0, 0, None, None, None, 1000) != 0
    assert lib.ls_stream_inject_copy_error(None, 0, 5) == 22


# ---------------------------------------------------------------------------- argument errors
EINVAL, ENOTSUP, EBUSY = 22, 95, 16


def _buffers(**kw):
    """A valid-looking buffer block (fake non-null device pointers); bind validates the
    arguments before any HIP call, so the errors below are decided on the CPU."""
    from leanstream_amd._native import LayerBuffers

    f = dict(width=4096, group_size=64, batch=1, slot_capacity=58, cache_groups=192, staging_groups=0,
             physical_groups=192, queue_capacity=58, cache=0x1000, staging=None, scales=0x2000)
    f.update(kw)
    return LayerBuffers(**f)


@pytest.mark.parametrize("change,code", [
    (dict(width=0), EINVAL), (dict(width=4000), EINVAL), (dict(group_size=0), EINVAL),
    (dict(group_size=257), EINVAL), (dict(slot_capacity=0), EINVAL), (dict(physical_groups=0), EINVAL),
    (dict(scales=None), EINVAL), (dict(cache=None), EINVAL), (dict(staging_groups=4, staging=None), EINVAL),
    (dict(batch=0), ENOTSUP), (dict(batch=33), ENOTSUP), (dict(batch=8, group_size=32), ENOTSUP),
    (dict(slot_capacity=4096), EINVAL), (dict(width=12288), ENOTSUP),
])
def test_bind_rejects_bad_arguments(change, code):
    """HipBackend::bind validation (the Triton backend's bind and the CUDA enqueue validate
    the same geometry: backends/triton/enqueue.cpp:19-25, kernels/streaming_mlp.cu:87)."""
    lib = _native.library()
    h = lib.ls_hip_create()
    try:
        assert lib.ls_hip_bind(h, C.byref(_buffers(**change))) == code
    finally:
        lib.ls_hip_destroy(h)


def test_bind_and_enqueue_null_arguments():
    lib = _native.library()
    assert lib.ls_hip_bind(None, C.byref(_buffers())) == EINVAL
    h = lib.ls_hip_create()
    try:
        assert lib.ls_hip_bind(h, None) == EINVAL
        q = HostQueue(4)
        x = np.zeros(4096, np.uint16)
        y = np.zeros(4096, np.uint16)
        args = (0, 0, 1, x.ctypes.data, y.ctypes.data, None, None, 0)
        # no queue, bad mode, unbound backend: refused before any GPU work
        assert lib.ls_hip_enqueue(h, *args, None, 1) == EINVAL
        assert lib.ls_hip_enqueue(h, *args, C.byref(q.view), 3) == EINVAL
        assert lib.ls_hip_enqueue(h, *args, C.byref(q.view), 1) == EINVAL
        assert lib.ls_hip_enqueue(None, *args, C.byref(q.view), 1) == EINVAL
        q.close()
    finally:
        lib.ls_hip_destroy(h)


class _Span(C.Structure):
    _fields_ = [("data", C.c_void_p), ("size", C.c_size_t)]


_COMMIT = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, _Span)
_COMPLETE = C.CFUNCTYPE(C.c_bool, C.c_void_p, C.c_uint32)


class _ComputeBackend(C.Structure):
    """ComputeBackend (include/leanstream/runtime.h): context + five function pointers."""
    _fields_ = [("context", C.c_void_p), ("enqueue", C.c_void_p), ("complete", _COMPLETE), ("commit", _COMMIT),
                ("defer_commit", C.c_void_p), ("cancel", C.c_void_p)]


def test_compute_backend_view_commit_without_hook_is_unsupported():
    """Without the application's cache-installation hook, commit returns ENOTSUP (the
    Triton backend's behaviour, backends/triton/enqueue.cpp:45); a backend that never
    launched is complete."""
    lib = _native.library()
    h = lib.ls_hip_create()
    try:
        cb = _ComputeBackend()
        assert lib.ls_hip_compute_backend(h, C.byref(cb), C.sizeof(cb)) == 0
        assert cb.context and cb.enqueue and not cb.defer_commit and not cb.cancel
        assert cb.commit(cb.context, 0, _Span(None, 0)) == ENOTSUP
        assert cb.complete(cb.context, 0)
    finally:
        lib.ls_hip_destroy(h)


def test_chain_entry_points_refuse_without_gpu_work():
    """ls_hip_enqueue_chain and its companions on an unbound backend: argument errors, no
    launch; the ctypes block has the C layout."""
    lib = _native.library()
    assert C.sizeof(_native.ChainLayer) == 120
    h = lib.ls_hip_create()
    try:
        layers = (_native.ChainLayer * 2)()
        assert lib.ls_hip_enqueue_chain(h, layers, 2, None) == EINVAL     # unbound
        assert lib.ls_hip_enqueue_chain(h, None, 1, None) == EINVAL
        assert lib.ls_hip_enqueue_chain(h, layers, 0, None) == EINVAL
        assert lib.ls_hip_enqueue_chain(None, layers, 1, None) == EINVAL
        assert lib.ls_hip_set_chain_stamps(h, None, 0) == EINVAL
        assert lib.ls_hip_chain_workers(h) == 0
        assert lib.ls_hip_last_seq(h) == 0 and lib.ls_hip_done_seq(h) == 0
    finally:
        lib.ls_hip_destroy(h)
