"""Failures of streamed layers through Runtime / LayerStep / WeightManager / HostStagingIO on
the GPU, then recovery (the adversarial cases of LeanStream examples/end_to_end/main.cu:82-113):

* an invalid finalize list (a group id out of range): EINVAL;
* a failed transport copy (the role of the reference's injected read error): EIO.

Each failed layer must end with its code in the queue's error word, the launch's
completion observed before the step is aborted, no status bit (the kernel left through
the queue error, not a timeout), and no group executed that was not published (the
published groups executed at most once each). Afterwards the same decoder runs clean layers
-- the failed layer ids included -- and they match the oracle.

Also: a layer whose last group arrives after the host's deadline fails at once (the cancel
comes before the wait for the stream) and leaves no status bit behind; the layer epilogue of
a failed layer withholds its flags; the decoder does not change the backend's own commit.
"""
import ctypes as C
import time

import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.backend import Mapped
from leanstream_amd.streaming import StreamingDecode

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-2
EIO, EINVAL, ENOTSUP, ETIMEDOUT = 5, 22, 95, 110


class _Span(C.Structure):
    _fields_ = [("data", C.c_void_p), ("size", C.c_size_t)]


class _ComputeBackend(C.Structure):
    """ComputeBackend (include/leanstream/runtime.h): context + five function pointers."""
    _fields_ = [("context", C.c_void_p), ("enqueue", C.c_void_p), ("complete", C.c_void_p),
                ("commit", C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, _Span)), ("defer_commit", C.c_void_p),
                ("cancel", C.c_void_p)]


def log(msg):
    print(msg, flush=True)


def _compare(y, ref, what):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = float(np.abs(y - ref).max())
    log(f"{what}: rel_l2={rel:.3e} max_abs={mx:.3e}")
    assert rel <= REL_L2 and mx <= MAX_ABS, (rel, mx)


def _published_dests(sd):
    desc, idx, ctrl = sd.queue()
    ready = int(ctrl[0])
    return ctrl, {int(desc[i, 3]) for i in idx[:ready]}


def _check_failed_layer(torch, sd, rc, times, expected, what):
    log(f"{what}: rc={rc}")
    assert rc == expected
    torch.cuda.synchronize()
    ctrl, published = _published_dests(sd)
    assert int(ctrl[5]) == expected, "queue error word"
    assert times[0, 5] > 0, "completion of the launch observed before abort"
    assert sd.backend.status() == 0
    ex = sd.executions.cpu().numpy()
    executed = set(np.nonzero(ex)[0].tolist())
    assert np.all(ex <= 1), "a group executed twice"
    assert executed <= published, ("executed groups that were never published", executed - published)
    log(f"{what}: published {len(published)}, executed {len(executed)}")


def test_failed_layers_then_recovery(torch_gpu):
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    sd = StreamingDecode(sc, layers=3)
    try:
        n = sd.cfg.groups
        # layer 0: finalize with an id out of range
        log("case: invalid finalize (EINVAL)")
        bad = np.array(sd.ranks[0], dtype=np.int32)
        bad[-1] = n
        sd.set_final(0, bad)
        sd.executions.zero_()
        torch.cuda.synchronize()
        rc, times, _ = sd.try_run(0, 1)
        _check_failed_layer(torch, sd, rc, times, EINVAL, "invalid finalize")
        sd.set_final(0, sd.ranks[0])

        # layer 1: the copy of one ranked group fails
        log("case: transport copy error (EIO)")
        sd.inject_copy_error(int(sd.ranks[1][3]), EIO)
        sd.executions.zero_()
        torch.cuda.synchronize()
        rc, times, _ = sd.try_run(1, 1)
        _check_failed_layer(torch, sd, rc, times, EIO, "copy error")
        sd.inject_copy_error(0, 0)

        # recovery: every layer (the failed ones included) runs clean and matches the oracle
        log("case: recovery, layers 0..2")
        sd.executions.zero_()
        sd.y.zero_()
        torch.cuda.synchronize()
        for layer in range(3):
            rc, times, _ = sd.try_run(layer, 1)
            assert rc == 0, (layer, rc)
            assert times[0, 6] > 0
        torch.cuda.synchronize()
        assert sd.backend.status() == 0
        assert np.all(sd.executions.cpu().numpy() == 3)   # once per layer
        ys = sd.y.cpu().numpy()
        k = sd.cfg.active
        for layer in range(3):
            hl = sd.host_layer(layer)
            rows = synth.descriptors(hl.cfg, sd.ranks[layer])
            ref = oracle.layer(rows, k, hl.cache, hl.scales, hl.x, sd.cfg.width, sd.cfg.group_size, threads=8)
            _compare(ys[layer], ref["y32"], f"recovered layer {layer}")
    finally:
        sd.close()


def _oracle_y(sd, layer):
    hl = sd.host_layer(layer)
    rows = synth.descriptors(hl.cfg, sd.ranks[layer])
    return oracle.layer(rows, sd.cfg.active, hl.cache, hl.scales, hl.x, sd.cfg.width, sd.cfg.group_size,
                        threads=8)["y32"]


def test_host_deadline_then_clean_layer(torch_gpu):
    """The last ranked group of layer 0 arrives 4 s after the layer begins, the host's
    deadline is 200 ms: ls_stream_run returns ETIMEDOUT well before the device's own 2 s
    bounded wait could end (the queue's error word releases the waiting workgroups before
    the stream is drained), leaves no status bit, and the same layer on time then returns 0
    and matches the oracle, as does the next one."""
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    sd = StreamingDecode(sc, layers=2)
    try:
        late = int(sd.ranks[0][-1])
        on_time = sd.arrivals[0].copy()
        sd.arrivals[0, late] = 4_000_000_000
        log("case: last group arrives 4 s late, deadline 200 ms")
        t0 = time.monotonic()
        rc, times, _ = sd.try_run(0, 1, timeout_ms=200)
        took = time.monotonic() - t0
        log(f"deadline layer: rc={rc} took {took:.3f} s")
        assert rc == ETIMEDOUT
        assert took < 1.5, took
        assert times[0, 5] == 0, "completion was not observed before the deadline"
        torch.cuda.synchronize()
        assert sd.backend.status() == 0
        sd.arrivals[0] = on_time
        log("case: the same layer on time, then layer 1")
        sd.y.zero_()
        torch.cuda.synchronize()
        for layer in range(2):
            rc, times, _ = sd.try_run(layer, 1)
            assert rc == 0, (layer, rc)
            assert times[0, 6] > 0
        torch.cuda.synchronize()
        assert sd.backend.status() == 0
        ys = sd.y.cpu().numpy()
        for layer in range(2):
            _compare(ys[layer], _oracle_y(sd, layer), f"after the deadline, layer {layer}")
    finally:
        sd.close()


def test_failed_layer_epilogue_withholds_flags(torch_gpu):
    """With the layer epilogue installed, a layer that fails (invalid finalize list: the
    runtime fails the queue, the launch leaves early) gets neither its hidden flag nor the
    bell; the next clean layer gets both, and its hidden rows are fp16(residual + y) bit for
    bit."""
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    sd = StreamingDecode(sc, layers=1)
    flags = Mapped(2, np.uint32)   # hidden flag, bell (host-coherent)
    try:
        d, n = sd.cfg.width, sd.cfg.groups
        rng = np.random.default_rng(5)
        residual_h = rng.standard_normal(d).astype(np.float16)
        residual = torch.from_numpy(residual_h).cuda()
        hidden = torch.zeros(d, dtype=torch.float16, device="cuda")
        flags.host[:] = 0
        sd.backend.set_epilogue(residual, hidden, flags.ptr, bell=flags.ptr + 4)
        log("case: invalid finalize with the epilogue installed")
        bad = np.array(sd.ranks[0], dtype=np.int32)
        bad[-1] = n
        sd.set_final(0, bad)
        torch.cuda.synchronize()
        rc, _, _ = sd.try_run(0, 1)
        torch.cuda.synchronize()
        log(f"failed layer: rc={rc} flags={flags.host.tolist()}")
        assert rc == EINVAL
        assert flags.host.tolist() == [0, 0]
        log("case: clean layer")
        sd.set_final(0, sd.ranks[0])
        rc, _, _ = sd.try_run(0, 1)
        torch.cuda.synchronize()
        log(f"clean layer: rc={rc} flags={flags.host.tolist()}")
        assert rc == 0
        assert flags.host[0] != 0 and flags.host[1] == 1
        y = sd.y[0].cpu().numpy()
        want = oracle.publish_hidden(residual_h, y)
        assert np.array_equal(hidden.cpu().numpy().view(np.uint16), want.view(np.uint16))
        sd.backend.set_epilogue(None, None)
    finally:
        sd.close()
        flags.close()


def test_decoder_leaves_backend_commit_unchanged(torch_gpu):
    """The decoder commits its streamed layers without a cache-installation hook, but does
    not install one into the caller's backend: once the decoder is destroyed, the backend's
    own ComputeBackend view refuses commits without the hook (ENOTSUP), as before."""
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    sd = StreamingDecode(sc, layers=1)
    try:
        log("case: one streamed layer, then the backend's own commit")
        rc, _, _ = sd.try_run(0, 1)
        assert rc == 0
        torch.cuda.synchronize()
        sd.lib.ls_stream_destroy(sd.handle)
        sd.handle = None
        view = _ComputeBackend()
        assert sd.lib.ls_hip_compute_backend(sd.backend.context, C.byref(view), C.sizeof(view)) == 0
        assert view.commit(view.context, 0, _Span(None, 0)) == ENOTSUP
    finally:
        sd.close()
