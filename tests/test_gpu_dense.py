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


@pytest.mark.parametrize("key,rows", [("c1d32", None), ("c5", (0, 7, 16, 31))])
def test_dense_layer_matches_oracle(torch_gpu, key, rows):
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
        for b in (range(cfg.batch) if rows is None else rows):
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
