"""A Group2 layer at the Ministral-3 8B shape (H 4096, I 14336: 7168 groups of 2 neurons, 1434
active) loaded from a packed bundle on disk (qweights.bin / scales.bin / metadata.json,
leanstream_amd/weights.py) into HBM and computed by the HIP kernels, against the oracle on the
same bytes (relative L2 <= 1e-3, max-abs <= 2e-2 on the fp32 output), with exactly-once
execution."""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth, weights
from leanstream_amd.backend import MODE_PROGRESSIVE, NativeBackend, ReadyQueue

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-2


def log(msg):
    print(msg, flush=True)


def test_group2_ministral_layer_from_bundle(torch_gpu, tmp_path):
    torch = torch_gpu
    H, I, G = 4096, 14336, 2
    groups = I // G
    k = int(np.floor(0.2 * groups + 0.5))
    log(f"case: Group2 bundle H={H} I={I} groups={groups} active={k}")
    packed = synth.fill_bytes(groups * G * 3 * H // 2, 0x62A)
    scales = synth.uniform_f16(groups * G * 3 * (H // 128), 0x62B, 0.005, 0.02)
    weights.write_packed_bundle(tmp_path / "layer_00", packed, scales, H, I, bundle_size=G)
    b = weights.Bundle(tmp_path / "layer_00")
    assert (b.groups, b.group_bytes) == (groups, 3 * H)
    cache, sc = b.to_device()
    x_host = synth.normal_f16(H, 0x62C)
    x = torch.from_numpy(x_host.copy()).cuda()
    active = synth.rank_top_k(synth.normal_f64(groups, 0x62D).astype(np.float32), k)
    descs = np.zeros((k, 5), dtype=np.uint32)
    descs[:, 0] = descs[:, 1] = descs[:, 2] = active      # group = physical bundle, resident in the cache
    descs[:, 3] = np.arange(k)
    core = torch.from_numpy(descs.reshape(-1).astype(np.int32)).cuda()
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    y32 = torch.empty(H, dtype=torch.float32, device="cuda")
    hidden = torch.zeros(k * G, dtype=torch.int64, device="cuda")
    partial = torch.zeros(k * H, dtype=torch.float32, device="cuda")
    executions = torch.zeros(k, dtype=torch.int32, device="cuda")
    backend = NativeBackend()
    backend.bind(H, G, k, cache, sc, physical_groups=groups, cache_groups=groups, staging=cache,
                 staging_groups=groups, queue_capacity=1, hidden=hidden, partial=partial, y32=y32,
                 executions=executions, batch=1)
    q = ReadyQueue(1)
    q.reset(1)
    q.seal(0)
    stream = torch.cuda.current_stream().cuda_stream
    backend.enqueue(0, 0, 1, x, y, stream, core, k, q, MODE_PROGRESSIVE)
    torch.cuda.synchronize()
    assert backend.status() == 0
    assert np.all(executions.cpu().numpy() == 1)
    ref = oracle.layer(descs, k, np.asarray(b.qweights).reshape(-1), b.scales.reshape(-1), x_host, H, G, threads=8)
    got = y32.cpu().numpy().astype(np.float64)
    want = ref["y32"].astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    mx = float(np.abs(got - want).max())
    log(f"Group2 bundle: rel_l2={rel:.3e} max_abs={mx:.3e}")
    assert rel <= REL_L2 and mx <= MAX_ABS
    assert np.array_equal(y.cpu().numpy().view(np.uint16), got.astype(np.float32).astype(np.float16).view(np.uint16))
    backend.close()
    q.close()
