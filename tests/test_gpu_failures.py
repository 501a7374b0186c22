"""Failures of streamed layers through Runtime / LayerStep / WeightManager / HostStagingIO on
the GPU, then recovery (the adversarial cases of LeanStream examples/end_to_end/main.cu:82-113):

* an invalid finalize list (a group id out of range): EINVAL;
* a failed transport copy (the role of the reference's injected read error): EIO.

Each failed layer must end with its code in the queue's error word, the launch's
completion observed before the step is aborted, no status bit (the kernel left through
the queue error, not a timeout), and no group executed that was not published (the
published groups executed at most once each). Afterwards the same decoder runs clean layers
-- the failed layer ids included -- and they match the oracle.
"""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.streaming import StreamingDecode

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-2
EIO, EINVAL = 5, 22


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
