"""Dense batched path (batch 32, matrix cores) against the CPU oracle.

Every row of y32 is compared with the oracle run on that row of x (relative L2 <= 1e-3,
max-abs <= 2e-2, fp32 pre-rounding output); y is y32 rounded to fp16; every unit is
computed once. x is bf16; the oracle gets its exact fp16 value (the value the matrix
cores multiply).
"""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.workload import DeviceLayer

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-2


def log(msg):
    print(msg, flush=True)


def compare(y32, ref, what):
    y32 = np.asarray(y32, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rel = np.linalg.norm(y32 - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = float(np.abs(y32 - ref).max())
    log(f"{what}: rel_l2={rel:.3e} max_abs={mx:.3e}")
    assert rel <= REL_L2 and mx <= MAX_ABS, (rel, mx)


def test_device_bf16_generator_matches_host(torch_gpu):
    cfg = synth.CONFIGS["c1d32"]
    log(f"case: bf16 x generator {cfg.name}")
    layer = DeviceLayer(cfg)
    try:
        bits = layer.x.cpu().numpy().view(np.uint16)
        assert np.array_equal(bits, synth.normal_bf16(cfg.batch * cfg.width, cfg.sub_seed(synth.SEED_X)))
    finally:
        layer.close()


@pytest.mark.parametrize("key", ["c1d32", "c5"])
def test_dense_layer_matches_oracle(torch_gpu, key):
    torch = torch_gpu
    cfg = synth.CONFIGS[key]
    log(f"case: dense layer {cfg.name} k={cfg.active} batch={cfg.batch}")
    layer = DeviceLayer(cfg)
    try:
        layer.seal_empty_queue(1)
        layer.run_core(epoch=1)
        torch.cuda.synchronize()
        assert layer.backend.status() == 0, layer.backend.status()
        d = cfg.width
        y32 = layer.y32.cpu().numpy().reshape(cfg.batch, d)
        y16 = layer.y.cpu().numpy().reshape(cfg.batch, d)
        assert np.all(np.isfinite(y32))
        assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16))
        assert np.all(layer.executions.cpu().numpy() == 1)
        hl = synth.host_layer(cfg)
        desc = layer.core_rows[0]
        for b in range(cfg.batch):
            ref = oracle.layer(desc, len(desc), hl.cache, hl.scales, hl.x[b * d:(b + 1) * d], d, cfg.group_size,
                               threads=8)
            compare(y32[b], ref["y32"], f"{cfg.name} row {b}")
        # a second launch (the other ring slot): identical bits
        layer.run_core(epoch=1)
        torch.cuda.synchronize()
        assert layer.backend.status() == 0
        assert np.array_equal(layer.y32.cpu().numpy().reshape(cfg.batch, d).view(np.uint32), y32.view(np.uint32))
    finally:
        layer.close()


def test_dense_launch_without_core_groups_then_with(torch_gpu):
    """A dense launch with no core units (only the reduction kernel runs) followed by a launch
    with core units: both complete (each launch leaves the next one's ring slot clear),
    y is 0 for the empty launch and matches the normal layer afterwards."""
    torch = torch_gpu
    cfg = synth.CONFIGS["c1d32"]
    log("case: dense launch with 0 core groups, then with core groups")
    layer = DeviceLayer(cfg)
    try:
        layer.seal_empty_queue(1)
        layer.run_core(epoch=1)
        torch.cuda.synchronize()
        want = layer.y32.cpu().numpy().copy()
        stream = torch.cuda.current_stream().cuda_stream
        for rep in range(2):
            layer.backend.enqueue(0, 0, 1, layer.x, layer.y, stream, None, 0, layer.queue)
            torch.cuda.synchronize()
            assert layer.backend.complete() and layer.backend.status() == 0
            assert not np.any(layer.y32.cpu().numpy())
            layer.run_core(epoch=1)
            torch.cuda.synchronize()
            assert layer.backend.complete() and layer.backend.status() == 0
            assert np.array_equal(layer.y32.cpu().numpy(), want)
    finally:
        layer.close()


def test_dense_launch_flags_published_queue_entries(torch_gpu):
    """The dense path computes resident groups only: a layer whose queue holds published
    entries is reported (LS_STATUS_QUEUE_UNCONSUMED) instead of silently lacking them."""
    from leanstream_amd.backend import STATUS_QUEUE_UNCONSUMED

    torch = torch_gpu
    cfg = synth.CONFIGS["c1d32"]
    log("case: dense launch with a non-empty ready queue")
    layer = DeviceLayer(cfg, queue_capacity=4)
    try:
        rows = synth.descriptors(cfg, layer.logical[:2], source_kind=0)
        q = layer.queue
        q.write_descriptors(rows)
        q.reset(2)
        q.seal(2)
        q.publish(0)
        q.publish(1)
        layer.run_core(epoch=2)
        torch.cuda.synchronize()
        assert layer.backend.complete()
        assert layer.backend.status() & STATUS_QUEUE_UNCONSUMED, layer.backend.status()
        layer.backend.clear_status()
        layer.seal_empty_queue(3)
        layer.run_core(epoch=3)
        torch.cuda.synchronize()
        assert layer.backend.status() == 0
    finally:
        layer.close()
