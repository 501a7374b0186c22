"""Layer chains on the GPU (ls_hip_enqueue_chain): one persistent launch over several layers.
Layer i's hidden state fp16(residual_i + y_i) (the epilogue's publication, LeanStream
backends/triton/reduction.py:17-22) is layer i + 1's residual and, through RMSNorm times the
layer's weight (examples/ministral/native/predictor_shared_input.cu:16-41), its input.

Every layer is checked on its own input: y32 against the oracle within the stated tolerance
(rel-L2 <= 1e-3, max-abs <= 2e-2), y = fp16(y32), the hidden state bit for bit against the
oracle's publication, and y32 bit for bit against the single-layer fused launch fed the
oracle's RMSNorm of the previous hidden state (both accumulate in the same fixed point, so
any bit of the in-kernel norm that differed from the oracle's would show). Also: per-layer
completion word, flags and bell; chains launched back to back give the bits of one longer
chain (the accumulators reset themselves across launches); a bad descriptor in a middle layer
ends the launch with a status bit and no hang, and the next chain is clean."""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.backend import STATUS_BAD_DESCRIPTOR, Mapped
from leanstream_amd.workload import DeviceLayer

pytestmark = pytest.mark.gpu

TOL_REL, TOL_ABS = 1e-3, 2e-2


def log(msg):
    print(msg, flush=True)


def stream(torch):
    return torch.cuda.current_stream().cuda_stream


def check_layers(torch, layer, order, outputs, x0, norm=None, eps=1e-5):
    """Every layer of a finished chain against the oracle and the fused launch."""
    y, y32, hidden = (t.cpu().numpy() for t in outputs)
    w = norm.cpu().numpy() if norm is not None else None
    cfg = layer.cfg
    x = x0.cpu().numpy()
    residual = x
    for i, c in enumerate(order):
        if i:
            residual = hidden[i - 1]
            x = oracle.rmsnorm(residual, w[i], eps) if w is not None else residual
        rows, cache, scales = layer.copy_rows(c)
        ref = oracle.layer(rows, len(rows), cache, scales, x, cfg.width, cfg.group_size, threads=8)
        r = ref["y32"].astype(np.float64)
        g = y32[i].astype(np.float64)
        rel = np.linalg.norm(g - r) / np.linalg.norm(r)
        mx = np.abs(g - r).max()
        log(f"  layer {i} (copy {c}): rel_l2={rel:.2e} max_abs={mx:.2e}")
        assert rel <= TOL_REL and mx <= TOL_ABS, (i, rel, mx)
        assert np.array_equal(y[i].view(np.uint16), y32[i].astype(np.float16).view(np.uint16)), i
        want = oracle.publish_hidden(residual, y[i])
        assert np.array_equal(hidden[i].view(np.uint16), want.view(np.uint16)), i
        # the fused single-layer launch on the same input gives the same fixed-point sums
        layer.x.copy_(torch.from_numpy(x).cuda())
        layer.seal_empty_queue(1000 + i)
        layer.run_core(copy=c, epoch=1000 + i)
        torch.cuda.synchronize()
        assert layer.backend.status() == 0
        assert np.array_equal(layer.y32.cpu().numpy().view(np.uint32), y32[i].view(np.uint32)), i


@pytest.mark.parametrize("key,copies,count", [("c1", 3, 8), ("c2", 2, 4)])
def test_chain_matches_oracle_every_layer(torch_gpu, key, copies, count):
    torch = torch_gpu
    cfg = synth.CONFIGS[key]
    log(f"case: chain {cfg.name} copies={copies} layers={count}")
    layer = DeviceLayer(cfg, copies=copies, diagnostics=False)
    order = [i % copies for i in range(count)]
    outputs = layer.chain_outputs(count)
    flags = Mapped(count + 1, np.uint32)
    flags.host[:] = 0
    x0 = layer.x.clone()
    norm = layer.chain_norm_weights(count)
    blocks = layer.chain_layers(order, outputs, x=x0, epoch0=5, flags=(flags.ptr, flags.ptr + 4 * count), norm=norm)
    layer.backend.enqueue_chain(blocks, stream(torch))
    torch.cuda.synchronize()
    assert layer.backend.status() == 0
    assert layer.backend.done_seq == layer.backend.last_seq
    assert layer.backend.complete()
    assert flags.host[:count].tolist() == [5 + i for i in range(count)]
    assert int(flags.host[count]) == count
    check_layers(torch, layer, order, outputs, x0, norm)
    layer.close()
    flags.close()


def test_chains_back_to_back_equal_one_longer_chain(torch_gpu):
    torch = torch_gpu
    cfg = synth.CONFIGS["c1"]
    log(f"case: chains back to back {cfg.name}")
    layer = DeviceLayer(cfg, copies=4, diagnostics=False)
    order = [0, 1, 2, 3, 0, 1, 2, 3, 1]
    long_out = layer.chain_outputs(len(order))
    x0 = layer.x.clone()
    norm = layer.chain_norm_weights(len(order))
    eps = 1e-5
    layer.backend.enqueue_chain(layer.chain_layers(order, long_out, x=x0, norm=norm, eps=eps), stream(torch))
    # the same layers as three launches of 3: each later launch starts from the previous one's
    # hidden state (its residual) and the oracle's RMSNorm of it (its input)
    parts = [layer.chain_outputs(3) for _ in range(3)]
    x, residual = x0, None
    for j, part in enumerate(parts):
        layer.backend.enqueue_chain(layer.chain_layers(order[3 * j:3 * j + 3], part, x=x, residual=residual,
                                                       norm=norm[3 * j:3 * j + 3], eps=eps), stream(torch))
        torch.cuda.synchronize()
        residual = part[2][2].clone()
        x = torch.from_numpy(oracle.rmsnorm(residual.cpu().numpy(), norm[3 * j + 3].cpu().numpy()
                                            if 3 * j + 3 < len(order) else norm[0].cpu().numpy(), eps)).cuda()
    torch.cuda.synchronize()
    assert layer.backend.status() == 0
    for j, part in enumerate(parts):
        for t in range(3):
            assert torch.equal(part[t], long_out[t][3 * j:3 * j + 3]), (j, t)
    layer.close()


def test_chain_bad_descriptor_fails_fast_then_recovers(torch_gpu):
    torch = torch_gpu
    cfg = synth.CONFIGS["c1"]
    log(f"case: chain bad descriptor {cfg.name}")
    layer = DeviceLayer(cfg, copies=2, diagnostics=False)
    layer.backend.set_spin_limit(20_000_000)   # 200 ms: nothing may wait on the failed layer for long
    bad = layer.core.clone()
    words = bad.view(-1, 5)
    words[layer.k + 3, 2] = 1 << 30            # copy 1, unit 3: source slot beyond the arena
    order = [0, 1, 0]
    outputs = layer.chain_outputs(3)
    blocks = layer.chain_layers(order, outputs)
    blocks[1]["core"] = bad.data_ptr() + layer.k * 20
    layer.backend.enqueue_chain(blocks, stream(torch))
    torch.cuda.synchronize()
    assert layer.backend.status() & STATUS_BAD_DESCRIPTOR
    assert layer.backend.done_seq == layer.backend.last_seq
    layer.backend.clear_status()
    layer.backend.set_spin_limit(200_000_000)
    x0 = layer.x.clone()
    norm = layer.chain_norm_weights(3)
    layer.backend.enqueue_chain(layer.chain_layers(order, outputs, x=x0, norm=norm), stream(torch))
    torch.cuda.synchronize()
    assert layer.backend.status() == 0
    check_layers(torch, layer, order, outputs, x0, norm)
    layer.close()
