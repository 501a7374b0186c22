"""The persistent launch on a few workers (ls_hip_set_workers) gives the bits of the full grid:
every wave then walks hundreds of items, so the staged walk's two slots alternate, descriptors
are fetched again every few items and down items wait for h published by the same workgroup's
other waves. The column sums are integers, so y does not depend on how the items were dealt.
Every descriptor still runs exactly once."""
import numpy as np
import pytest

from leanstream_amd import synth
from leanstream_amd.backend import MODE_PROGRESSIVE
from leanstream_amd.workload import DeviceLayer

from test_gpu_parity import _queue_run, log, sync_and_check_status

pytestmark = pytest.mark.gpu

G8 = synth.LayerConfig("sparse_int4_mlp_d1024_f4096_g8_a20", 1024, 4096, 0.20, group_size=8, seed=0x6808)


def _core_bits(torch, layer):
    layer.executions.zero_()
    layer.seal_empty_queue(1)
    layer.run_core(epoch=1)
    sync_and_check_status(torch, layer)
    assert np.all(layer.executions.cpu().numpy() == 1)
    return layer.y32.cpu().numpy().view(np.uint32).copy(), layer.y.cpu().numpy().view(np.uint16).copy()


@pytest.mark.parametrize("key", ["c1", "c2", "c4", "c1b4", "g8"])
def test_few_workers_give_the_full_grid_bits(torch_gpu, key):
    torch = torch_gpu
    cfg = G8 if key == "g8" else synth.CONFIGS[key]
    log(f"case: few workers {cfg.name}")
    layer = DeviceLayer(cfg)
    try:
        full = _core_bits(torch, layer)
        for workers in (1, 3, 17):
            log(f"  workers {workers}")
            layer.backend.set_workers(workers)
            got = _core_bits(torch, layer)
            assert np.array_equal(got[0], full[0]) and np.array_equal(got[1], full[1]), workers
        layer.backend.set_workers(0)
        assert all(np.array_equal(a, b) for a, b in zip(_core_bits(torch, layer), full))
    finally:
        layer.close()


def test_few_workers_consume_the_ready_queue(torch_gpu):
    torch = torch_gpu
    cfg = synth.CONFIGS["c2"]
    log(f"case: few workers, ready queue {cfg.name}")
    layer = DeviceLayer(cfg)
    try:
        k = len(layer.logical)
        _queue_run(torch, layer, k // 3, MODE_PROGRESSIVE, "delayed", epoch=3)
        want = layer.y32.cpu().numpy().view(np.uint32).copy()
        layer.backend.set_workers(5)
        layer.executions.zero_()
        _queue_run(torch, layer, k // 3, MODE_PROGRESSIVE, "delayed", epoch=4)
        assert np.all(layer.executions.cpu().numpy()[:k] == 1)
        assert np.array_equal(layer.y32.cpu().numpy().view(np.uint32), want)
    finally:
        layer.close()
