"""Every width the library is built for, on each kernel family that serves it, against the
oracle: d = 256, 512 and 2048 beside the 1024, 4096 and 8192 of the named workloads.

- staged walk (64-neuron groups, batch 1), with its 64-column quarters where every item of a
  range gets a wave of its own;
- plain walk at batch 4 (down tiles shared by the rows);
- plain walk with 128-neuron groups (two 64-row passes per down tile);
- packed walk (8-neuron groups: a down item spans the rows of 8 core units);
- batch 2 and 3 on the batch-4 kernels;
- dense batched path (batch 5 .. 32, bf16 x, matrix cores);
- the ready queue (a third of the units resident, the rest published while the launch runs);
- the split entry point (stage A, stage B, reduction) at batch 4, bit for bit the fused launch.

Bars as in the other parity tests: relative L2 <= 1e-3 and max-abs <= 2e-2 on the fp32 output,
the fp16 output the round-to-nearest of it, h per neuron, every descriptor executed once.
"""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.backend import MODE_PROGRESSIVE
from leanstream_amd.workload import DeviceLayer

from test_gpu_parity import _queue_run, check_h, compare, log, sync_and_check_status

pytestmark = pytest.mark.gpu


def config(d, G=64, batch=1, dense=False):
    ffn = 4 * d
    kind = "dense" if dense else "sparse"
    return synth.LayerConfig(f"{kind}_int4_mlp_d{d}_f{ffn}_g{G}_b{batch}", d, ffn, 1.0 if dense else 0.25,
                             group_size=G, batch=batch, selection="all" if dense else "ranking",
                             x_dtype="bf16" if dense else "f16", seed=0x3D00 + d + G + batch)


def check_rows(layer, rows, what):
    """Every batch row of y (and h) against the oracle on that row of x."""
    cfg = layer.cfg
    d = cfg.width
    hl = synth.host_layer(cfg)
    y32 = layer.y32.cpu().numpy().reshape(cfg.batch, d)
    y16 = layer.y.cpu().numpy().reshape(cfg.batch, d)
    h = layer.hidden_h() if cfg.batch <= 4 else None
    for b in range(cfg.batch):
        ref = oracle.layer(rows, int(rows[:, 3].max()) + 1, hl.cache, hl.scales, hl.x[b * d:(b + 1) * d], d,
                           cfg.group_size, threads=8)
        compare(y32[b], ref["y32"], f"{what} row {b}")
        assert np.array_equal(y16[b].view(np.uint16), y32[b].astype(np.float16).view(np.uint16))
        if h is not None:
            check_h(h[:, b, :] if h.ndim == 3 else h, ref["h"], f"{what} row {b} h")


CASES = [(256, 64, 1), (512, 64, 1), (2048, 64, 1),       # staged walk
         (256, 64, 4), (512, 64, 4), (2048, 64, 4),       # plain walk, batch 4
         (1024, 128, 1), (2048, 128, 1),                  # plain walk, two-pass down tiles
         (512, 8, 1), (2048, 8, 1),                       # packed walk
         (1024, 64, 2), (1024, 64, 3), (8192, 64, 3)]     # batch 2 and 3 on the batch-4 kernels


@pytest.mark.parametrize("d,G,batch", CASES)
def test_core_layer_at_every_width(torch_gpu, d, G, batch):
    torch = torch_gpu
    cfg = config(d, G, batch)
    log(f"case: core layer {cfg.name} k={cfg.active}")
    layer = DeviceLayer(cfg)
    try:
        layer.seal_empty_queue(1)
        layer.run_core(epoch=1)
        sync_and_check_status(torch, layer)
        check_rows(layer, layer.core_rows[0], cfg.name)
        assert np.all(layer.executions.cpu().numpy() == 1)
    finally:
        layer.close()


@pytest.mark.parametrize("d,batch", [(512, 32), (2048, 32), (1024, 5), (1024, 19)])
def test_dense_layer_at_other_widths(torch_gpu, d, batch):
    """Other widths, and batches below 32 (rows >= batch of x16 and h16 are zero)."""
    torch = torch_gpu
    cfg = config(d, batch=batch, dense=True)
    log(f"case: dense layer {cfg.name} k={cfg.active}")
    layer = DeviceLayer(cfg)
    try:
        layer.seal_empty_queue(1)
        layer.run_core(epoch=1)
        sync_and_check_status(torch, layer)
        check_rows(layer, layer.core_rows[0], cfg.name)
        assert np.all(layer.executions.cpu().numpy() == 1)
    finally:
        layer.close()


@pytest.mark.parametrize("d,G", [(512, 64), (2048, 64), (2048, 8)])
def test_queue_units_at_other_widths(torch_gpu, d, G):
    torch = torch_gpu
    cfg = config(d, G)
    log(f"case: queue units {cfg.name} k={cfg.active}")
    layer = DeviceLayer(cfg)
    try:
        k = len(layer.logical)
        layer.executions.zero_()
        rows, _ = _queue_run(torch, layer, k // 3, MODE_PROGRESSIVE, "delayed", epoch=5)
        check_rows(layer, rows, f"{cfg.name} queue")
        assert np.all(layer.executions.cpu().numpy()[:k] == 1)
    finally:
        layer.close()


@pytest.mark.parametrize("d", [1024, 2048])
def test_split_entry_point_at_batch_4_matches_fused(torch_gpu, d):
    """The reference's three-launch split (stage A, stage B, reduction; candidate 4) at batch 4:
    the same bits as the fused launch, resident-only and with a third of the units resident and
    the rest published while stage B runs (integer column sums: entry-point independent)."""
    torch = torch_gpu
    cfg = config(d, 64, 4)
    log(f"case: split entry point {cfg.name} k={cfg.active}")
    out = {}
    for name, table in (("fused", None), ("split", [[4]])):
        layer = DeviceLayer(cfg, offline_table=table)
        try:
            layer.seal_empty_queue(1)
            layer.run_core(epoch=1)
            sync_and_check_status(torch, layer)
            if table:
                assert layer.backend.last_candidate() == 4
            out[name, "core"] = (layer.y32.cpu().numpy().copy(), layer.y.cpu().numpy().copy())
            assert np.all(layer.executions.cpu().numpy() == 1)
            k = len(layer.logical)
            layer.executions.zero_()
            rows, _ = _queue_run(torch, layer, k // 3, MODE_PROGRESSIVE, "delayed", epoch=3)
            out[name, "queue"] = (layer.y32.cpu().numpy().copy(), layer.y.cpu().numpy().copy())
            assert np.all(layer.executions.cpu().numpy()[:k] == 1)
            if name == "split":
                check_rows(layer, rows, f"{cfg.name} split queue")
        finally:
            layer.close()
    for run in ("core", "queue"):
        for a, b in zip(out["fused", run], out["split", run]):
            assert np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else np.uint16),
                                  b.view(np.uint32 if b.dtype == np.float32 else np.uint16)), run
