"""Groups of at most 32 neurons (LeanStream's Ministral-3 8B pack has 2-neuron groups,
examples/ministral/pack/pack_mistral.py) on the packed kernels: a down item of the resident
range covers the rows of 64 / G consecutive core units, queue units keep one down item each.

Checked against the CPU oracle (relative L2 <= 1e-3, max-abs <= 2e-2 on y32; y16 is the
round-to-nearest of y32), per-neuron h, exactly-once execution per descriptor, and bit-exact
equality where the reference's own tests require it (persistent_mlp_test.cu:64-67): across
consumer modes and publication orders for one core/queue split, across repeated launches, and
between the fused and the split entry points.
"""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.backend import MODE_BATCH_COMPAT, MODE_PROGRESSIVE
from leanstream_amd.workload import DeviceLayer

from test_gpu_parity import check_h, compare, log

pytestmark = pytest.mark.gpu

# d_model 1024; G = 3 leaves a pack of 21 units (63 rows)
FFN = {2: 4096, 3: 3072, 8: 4096, 32: 4096}


def config(G):
    return synth.LayerConfig(f"sparse_int4_mlp_d1024_f{FFN[G]}_g{G}_a20", 1024, FFN[G], 0.20, group_size=G,
                             seed=0x5A11 + G)


def reference(cfg, rows):
    hl = synth.host_layer(cfg)
    return oracle.layer(rows, int(rows[:, 3].max()) + 1, hl.cache, hl.scales, hl.x, cfg.width, cfg.group_size,
                        threads=8)


def run_queue(torch, layer, core_n, mode, order, epoch, delayed, entry=None):
    """core_n resident groups, the rest through the ready queue published in `order`."""
    cfg = layer.cfg
    core_rows = synth.descriptors(cfg, layer.logical[:core_n])
    q_rows = synth.descriptors(cfg, layer.logical[core_n:], dest_base=core_n)
    total = len(q_rows)
    core_dev = torch.from_numpy(core_rows.reshape(-1).astype(np.int32)).cuda() if core_n else None
    q = layer.queue
    q.write_descriptors(q_rows)
    q.reset(epoch)
    stream = torch.cuda.current_stream().cuda_stream
    if not delayed:
        q.seal(total)
        for i in order:
            q.publish(int(i))
    layer.backend.enqueue(0, 0, epoch, layer.x, layer.y, stream, core_dev, core_n, q, mode)
    if delayed:
        q.seal(total)
        q.start_publisher(order, np.arange(total, dtype=np.uint64) * 20_000).join()
    torch.cuda.synchronize()
    assert layer.backend.status() == 0, layer.backend.status()
    assert q.words()["ready_count"] == total
    if entry is not None:
        assert layer.backend.last_candidate() == entry
    return np.concatenate([core_rows, q_rows]) if core_n else q_rows


@pytest.mark.parametrize("G", sorted(FFN))
def test_small_group_core_layer_matches_oracle(torch_gpu, G):
    torch = torch_gpu
    cfg = config(G)
    log(f"case: packed core layer {cfg.name} k={cfg.active} (packs of {64 // G} units)")
    layer = DeviceLayer(cfg)
    layer.seal_empty_queue(1)
    layer.run_core(epoch=1)
    torch.cuda.synchronize()
    assert layer.backend.status() == 0, layer.backend.status()
    rows = layer.core_rows[0]
    ref = reference(cfg, rows)
    y32 = layer.y32.cpu().numpy().copy()
    compare(y32, ref["y32"], cfg.name)
    assert np.array_equal(layer.y.cpu().numpy().view(np.uint16), y32.astype(np.float16).view(np.uint16))
    check_h(layer.hidden_h(), ref["h"], "h")
    assert np.all(layer.executions.cpu().numpy() == 1)
    # the same launch again: same packs, same bits; every descriptor executed once more
    layer.seal_empty_queue(2)
    layer.run_core(epoch=2)
    torch.cuda.synchronize()
    assert layer.backend.status() == 0
    assert np.array_equal(layer.y32.cpu().numpy(), y32)
    assert np.all(layer.executions.cpu().numpy() == 2)
    layer.close()


@pytest.mark.parametrize("G", [2, 3])
def test_small_group_queue_modes_and_orders_bit_exact(torch_gpu, G):
    torch = torch_gpu
    cfg = config(G)
    log(f"case: packed kernels, queue paths {cfg.name}")
    layer = DeviceLayer(cfg)
    k = len(layer.logical)
    outs = {}
    for core_n in (0, k // 3):
        total = k - core_n
        order = synth.ready_order(total, cfg)
        runs = [("progressive_delayed", MODE_PROGRESSIVE, order, True),
                ("progressive_before", MODE_PROGRESSIVE, order, False),
                ("batch_delayed", MODE_BATCH_COMPAT, order, True),
                ("reversed_order", MODE_PROGRESSIVE, order[::-1].copy(), True)]
        for name, mode, ordr, delayed in runs:
            log(f"  core {core_n}: {name}")
            layer.executions.zero_()
            rows = run_queue(torch, layer, core_n, mode, ordr, epoch=7, delayed=delayed)
            outs[(core_n, name)] = layer.y32.cpu().numpy().copy()
            assert np.all(layer.executions.cpu().numpy() == 1)
        ref = reference(cfg, rows)
        compare(outs[(core_n, "progressive_delayed")], ref["y32"], f"{cfg.name} core {core_n}")
        base = outs[(core_n, "progressive_delayed")]
        for name, *_ in runs:
            assert np.array_equal(outs[(core_n, name)], base), (core_n, name)
    layer.close()
    log("  split entry point, same core/queue split")
    split = DeviceLayer(cfg, offline_table=[[4]])
    order = synth.ready_order(k - k // 3, cfg)
    run_queue(torch, split, k // 3, MODE_PROGRESSIVE, order, epoch=3, delayed=True, entry=4)
    assert np.array_equal(split.y32.cpu().numpy(), outs[(k // 3, "progressive_delayed")])
    split.close()
