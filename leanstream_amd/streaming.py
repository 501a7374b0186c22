"""Streaming decode step over host-staged layers (ls_stream_* in include/leanstream_hip.h).

Every layer's packed groups live in one pinned host store (layer l, physical group p
at byte (l * groups + p) * group_bytes, the file offset of its GroupLayout). Per layer,
the native loop drives Runtime / LayerStep / WeightManager with HostStagingIO: the
ranked groups are copied into the device staging arena as they arrive (SDMA engines
driven directly, or hipMemcpyAsync on side streams), and each completion publishes READY to the persistent consumer that was
pre-enqueued for the layer. Scales of every layer stay in HBM (physical row
l * groups + p); x is shared by the layers, each layer writes its own y row.
"""
import ctypes as C

import numpy as np

from . import _native, synth
from .backend import MODE_PROGRESSIVE, NativeBackend
from ._native import DeviceQueue, GroupLayout, StreamLayer, StreamSetup

COPY_SDMA, COPY_HIP = 0, 1
TIME_FIELDS = ("begin", "begun", "updated", "enqueued", "finalized", "complete", "committed")


def _check(rc, what):
    if rc:
        raise RuntimeError(f"{what} failed: {rc}")


class StreamingDecode:
    def __init__(self, sc, layers=None, qd=24, copy_engine=COPY_SDMA, copy_queues=8, copy_chunk=0,
                 mode=MODE_PROGRESSIVE, arrivals=True):
        import torch

        self.torch = torch
        self.sc = sc
        cfg = sc.layer
        self.cfg = cfg
        self.layers = L = sc.layers if layers is None else int(layers)
        lib = self.lib = _native.library()
        dev = torch.device("cuda")
        n, G, d, gb = cfg.groups, cfg.group_size, cfg.width, cfg.group_bytes
        stream = torch.cuda.current_stream().cuda_stream
        self.host = torch.empty(L * n * gb, dtype=torch.uint8, pin_memory=True)
        self.scales = torch.empty(L * n * cfg.scale_words, dtype=torch.float16, device=dev)
        tmp = torch.empty(n * gb, dtype=torch.uint8, device=dev)
        for l in range(L):
            lc = sc.layer_config(l)
            _check(lib.ls_synth_bytes(tmp.data_ptr(), n * gb, lc.sub_seed(synth.SEED_W), stream), "synth bytes")
            self.host[l * n * gb:(l + 1) * n * gb].copy_(tmp)
            _check(lib.ls_synth_uniform_f16(self.scales.data_ptr() + 2 * l * n * cfg.scale_words, n * cfg.scale_words,
                                            lc.sub_seed(synth.SEED_S), cfg.scale_lo, cfg.scale_hi, stream),
                   "synth scales")
        torch.cuda.synchronize()
        del tmp
        self.x = torch.empty(cfg.batch * d, dtype=torch.float16, device=dev)
        _check(lib.ls_synth_normal_f16(self.x.data_ptr(), cfg.batch * d, sc.x_config().sub_seed(synth.SEED_X),
                                       stream), "synth x")
        self.y = torch.zeros(L, cfg.batch * d, dtype=torch.float16, device=dev)
        self.staging = torch.zeros(n * gb, dtype=torch.uint8, device=dev)
        k = cfg.active
        self.y32 = torch.empty(cfg.batch * d, dtype=torch.float32, device=dev)
        self.hidden = torch.zeros(k * cfg.batch * G, dtype=torch.int64, device=dev)
        self.executions = torch.zeros(k, dtype=torch.int32, device=dev)
        self.backend = NativeBackend()
        self.backend.bind(d, G, k, None, self.scales, physical_groups=L * n, cache_groups=0, staging=self.staging,
                          staging_groups=n, queue_capacity=n, hidden=self.hidden, y32=self.y32,
                          executions=self.executions, batch=cfg.batch)
        # per-layer rank, layout and arrival tables
        self.ranks = [synth.stream_rank(sc, l) for l in range(L)]
        phys = synth.physical_of(np.arange(n), n)
        self.layouts = np.zeros(L * n, dtype=[("logical", "<u4"), ("physical", "<u4"), ("offset", "<u8"),
                                              ("bytes", "<u4"), ("reserved", "<u4")])
        for l in range(L):
            rows = self.layouts[l * n:(l + 1) * n]
            rows["logical"] = np.arange(n)
            rows["physical"] = l * n + phys
            rows["offset"] = (l * n + phys).astype(np.uint64) * gb
            rows["bytes"] = gb
        assert self.layouts.itemsize == C.sizeof(GroupLayout)
        self.rank_words = np.zeros((L, k), dtype=np.int32)
        for l in range(L):
            self.rank_words[l] = self.ranks[l]
        self.arrivals = np.zeros((L, n), dtype=np.uint64)
        if arrivals:
            for l in range(L):
                self.arrivals[l] = sc.arrivals(l, self.ranks[l])
        self.entries = (StreamLayer * L)()
        for l in range(L):
            e = self.entries[l]
            e.layout = self.layouts.ctypes.data + l * n * self.layouts.itemsize
            e.rank = self.rank_words.ctypes.data + l * k * 4
            e.rank_count = k
            e.final_ids = e.rank
            e.final_count = k
            e.arrival_ns = self.arrivals.ctypes.data + l * n * 8
            e.input = self.x.data_ptr()
            e.output = self.y.data_ptr() + l * cfg.batch * d * 2
        self.setup = StreamSetup(self.backend.context, self.host.data_ptr(), self.host.numel(), self.staging.data_ptr(),
                                 self.staging.numel(), gb, gb, n, L, qd, copy_engine, copy_queues, copy_chunk, mode,
                                 torch.cuda.current_device())
        torch.cuda.synchronize()
        self.handle = lib.ls_stream_create(C.byref(self.setup))
        if not self.handle:
            raise RuntimeError("ls_stream_create failed")

    def run(self, first=0, count=None, timeout_ms=10000):
        """Run layers [first, first + count); returns (times [count, 7] ns from the call's
        start, stamps [count, groups, 3] ns from each layer's begin)."""
        rc, times, stamps = self.try_run(first, count, timeout_ms)
        _check(rc, "ls_stream_run")
        return times, stamps

    def try_run(self, first=0, count=None, timeout_ms=10000):
        """As run, returning (return code, times, stamps) instead of raising."""
        count = self.layers - first if count is None else count
        n = self.cfg.groups
        times = np.zeros((count, 7), dtype=np.uint64)
        stamps = np.zeros((count, n, 3), dtype=np.uint64)
        stream = self.torch.cuda.current_stream().cuda_stream
        entries = C.cast(C.byref(self.entries, first * C.sizeof(StreamLayer)), C.c_void_p)
        rc = self.lib.ls_stream_run(self.handle, entries, count, first, stream, times.ctypes.data, stamps.ctypes.data,
                                    timeout_ms)
        return rc, times, stamps

    def inject_copy_error(self, group, error):
        """Refuse every copy of logical group `group` with `error` (0 clears)."""
        _check(self.lib.ls_stream_inject_copy_error(self.handle, group, error), "ls_stream_inject_copy_error")

    def set_final(self, layer, ids):
        """Replace layer `layer`'s final list (finalize argument) with `ids`."""
        self._finals = getattr(self, "_finals", {})
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        self._finals[layer] = arr
        self.entries[layer].final_ids = arr.ctypes.data
        self.entries[layer].final_count = len(arr)

    def queue(self):
        """(descriptors [capacity, 5], ready_indices [capacity], control words [32]) as numpy copies."""
        q = DeviceQueue()
        _check(self.lib.ls_stream_queue(self.handle, C.byref(q)), "ls_stream_queue")
        cap = q.capacity
        desc = np.ctypeslib.as_array((C.c_uint32 * (5 * cap)).from_address(q.descriptors)).reshape(cap, 5).copy()
        idx = np.ctypeslib.as_array((C.c_uint32 * cap).from_address(q.ready_indices)).copy()
        ctrl = np.ctypeslib.as_array((C.c_uint32 * 32).from_address(q.control)).copy()
        return desc, idx, ctrl

    def host_layer(self, l):
        """Host copy of layer l in the oracle's layout (cache in physical order, scales, x)."""
        cfg, n = self.cfg, self.cfg.groups
        cache = self.host[l * n * cfg.group_bytes:(l + 1) * n * cfg.group_bytes].numpy().copy()
        scales = self.scales[l * n * cfg.scale_words:(l + 1) * n * cfg.scale_words].cpu().numpy()
        return synth.HostLayer(self.sc.layer_config(l), cache, scales, self.x.cpu().numpy())

    def close(self):
        self.torch.cuda.synchronize()
        if self.handle:
            self.lib.ls_stream_destroy(self.handle)
            self.handle = None
        self.backend.close()
