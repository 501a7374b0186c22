"""The allocation-free resident layer (ls_hip_core_layer_noalloc) against ls_hip_enqueue on
the same inputs: y (fp16) and the fp32 y bit for bit, and a clean status word, over calls
in a row whose inputs shrink (a smaller width, then fewer groups), so that what one call
leaves in the library's shared array cannot reach the next call's output; one of the layers
has 8-neuron groups (the packed kernels), one has four batch rows."""
import numpy as np
import pytest

from leanstream_amd import _native, synth
from leanstream_amd.workload import DeviceLayer

EINVAL, ENOSPC, ENOTSUP = 22, 28, 95


def log(msg):
    print(msg, flush=True)


def _existing(torch, layer, count):
    """y and y32 of ls_hip_enqueue: `count` core descriptors, empty sealed queue."""
    layer.seal_empty_queue(1)
    stream = torch.cuda.current_stream().cuda_stream
    layer.backend.enqueue(0, 0, 1, layer.x, layer.y, stream, layer.core_ptr(0), count, layer.queue, 0)
    torch.cuda.synchronize()
    assert layer.backend.status() == 0
    return layer.y.clone(), layer.y32.clone()


def _noalloc(torch, lib, layer, count):
    cfg = layer.cfg
    y = torch.full_like(layer.y, 0x7BFF)                 # garbage the call must overwrite
    y32 = torch.full_like(layer.y32, float("nan"))
    status = torch.full((1,), -1, dtype=torch.int32, device=layer.y.device)
    groups = layer.copies * cfg.groups
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.ls_hip_core_layer_noalloc(cfg.width, cfg.group_size, cfg.batch, layer.cache.data_ptr(), groups,
                                       layer.scales.data_ptr(), groups, layer.core_ptr(0), count, layer.x.data_ptr(),
                                       y.data_ptr(), y32.data_ptr(), status.data_ptr(), stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    return y, y32


def _same_bits(a, b, what):
    ua = a.cpu().numpy().view(np.uint16 if a.element_size() == 2 else np.uint32)
    ub = b.cpu().numpy().view(np.uint16 if b.element_size() == 2 else np.uint32)
    assert np.array_equal(ua, ub), f"{what}: {np.count_nonzero(ua != ub)} words differ"


@pytest.mark.gpu
def test_noalloc_layer_matches_enqueue(torch_gpu):
    torch = torch_gpu
    lib = _native.library()
    # (config, core groups): each call smaller than the one before; "g8" (8-neuron groups,
    # d_model 1024) takes the packed kernels, whose down items span 8 units; "c1b4" is batch 4
    g8 = synth.LayerConfig("sparse_int4_mlp_d1024_f4096_g8_a20", 1024, 4096, 0.20, group_size=8, seed=0x6808)
    cases = [("c2", None), ("c1b4", None), ("g8", None), ("c1", None), ("c1", 5)]
    layers = {}
    for key, count in cases:
        cfg = g8 if key == "g8" else synth.CONFIGS[key]
        layer = layers.get(key) or DeviceLayer(cfg)
        layers[key] = layer
        k = layer.k if count is None else count
        log(f"case: noalloc {cfg.name} groups={k} of {layer.k}")
        ref_y, ref_y32 = _existing(torch, layer, k)
        y, y32 = _noalloc(torch, lib, layer, k)
        _same_bits(y32, ref_y32, f"{key}/{k} y32")
        _same_bits(y, ref_y, f"{key}/{k} y")
    for layer in layers.values():
        layer.close()


@pytest.mark.gpu
def test_noalloc_rejects_sizes_beyond_its_array(torch_gpu):
    torch = torch_gpu
    lib = _native.library()
    cfg = synth.CONFIGS["c1"]
    log("case: noalloc limits")
    layer = DeviceLayer(cfg)
    groups = layer.copies * cfg.groups
    y = torch.empty_like(layer.y)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.ls_hip_core_layer_noalloc(cfg.width, cfg.group_size, cfg.batch, layer.cache.data_ptr(), groups,
                                       layer.scales.data_ptr(), groups, layer.core_ptr(0), 1025, layer.x.data_ptr(),
                                       y.data_ptr(), None, None, stream)
    assert rc == ENOSPC
    layer.close()


@pytest.mark.parametrize("change,code", [
    (dict(width=0), EINVAL), (dict(width=1000), EINVAL), (dict(group_size=0), EINVAL), (dict(batch=0), EINVAL),
    (dict(cache=None), EINVAL), (dict(scales=None), EINVAL), (dict(cache_groups=0), EINVAL),
    (dict(core=None), EINVAL), (dict(x=None), EINVAL), (dict(y=None), EINVAL),
    (dict(batch=5), ENOTSUP), (dict(width=768), ENOTSUP),
    (dict(width=16384), ENOSPC), (dict(core_count=1025), ENOSPC), (dict(core_count=600, group_size=64), ENOSPC),
])
def test_noalloc_argument_errors_before_any_gpu_call(change, code):
    """Arguments are checked before the entry point touches HIP (fake device pointers)."""
    lib = _native.library()
    f = dict(width=4096, group_size=64, batch=1, cache=0x1000, cache_groups=192, scales=0x2000, scale_groups=192,
             core=0x3000, core_count=58, x=0x4000, y=0x5000)
    f.update(change)
    rc = lib.ls_hip_core_layer_noalloc(f["width"], f["group_size"], f["batch"], f["cache"], f["cache_groups"],
                                       f["scales"], f["scale_groups"], f["core"], f["core_count"], f["x"], f["y"],
                                       None, None, None)
    assert rc == code
