"""Every device wait is bounded: a layer whose epoch is never published ends with the
timeout status bit instead of hanging (the condition is forced from the host with a
short spin limit on the kernel's own bounded wait)."""
import ctypes as C
import time

import numpy as np
import pytest

from leanstream_amd import synth
from leanstream_amd.backend import MODE_PROGRESSIVE, STATUS_TIMEOUT
from leanstream_amd.workload import DeviceLayer

pytestmark = pytest.mark.gpu

ETIMEDOUT, ENOTSUP = 110, 95


class _Span(C.Structure):
    _fields_ = [("data", C.c_void_p), ("size", C.c_size_t)]


class _ComputeBackend(C.Structure):
    """ComputeBackend (include/leanstream/runtime.h): context + five function pointers."""
    _fields_ = [("context", C.c_void_p), ("enqueue", C.c_void_p), ("complete", C.c_void_p),
                ("commit", C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, _Span)), ("defer_commit", C.c_void_p),
                ("cancel", C.c_void_p)]


def test_unpublished_epoch_times_out(torch_gpu):
    torch = torch_gpu
    print("case: epoch never published, spin limit 20 ms", flush=True)
    cfg = synth.CONFIGS["c1"]
    layer = DeviceLayer(cfg)
    layer.backend.set_spin_limit(2_000_000)   # 20 ms of the 100 MHz device clock
    q = layer.queue
    q.write_descriptors(synth.descriptors(cfg, layer.logical))
    q.reset(7)   # epoch word stays 0: the consumer never sees epoch 7
    t0 = time.time()
    layer.backend.enqueue(0, 0, 7, layer.x, layer.y, torch.cuda.current_stream().cuda_stream, None, 0, q,
                          MODE_PROGRESSIVE)
    torch.cuda.synchronize()
    assert time.time() - t0 < 5.0
    assert layer.backend.status() & STATUS_TIMEOUT
    # the ComputeBackend view refuses to commit a layer whose launch timed out
    view = _ComputeBackend()
    assert layer.backend.lib.ls_hip_compute_backend(layer.backend.context, C.byref(view), C.sizeof(view)) == 0
    assert view.commit(view.context, 0, _Span(None, 0)) == ETIMEDOUT
    layer.backend.clear_status()
    assert view.commit(view.context, 0, _Span(None, 0)) == ENOTSUP   # no install hook: as before
    layer.backend.set_spin_limit(200_000_000)
    # the backend keeps working afterwards
    layer.seal_empty_queue(8)
    layer.run_core(epoch=8)
    torch.cuda.synchronize()
    assert layer.backend.status() == 0
    assert np.isfinite(layer.y32.cpu().numpy()).all()
    layer.close()
