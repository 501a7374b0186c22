"""The layer epilogue on the GPU (ls_hip_set_epilogue): next hidden state fp16(residual + y)
(LeanStream backends/triton/reduction.py:17-28) and its RMSNorm
(examples/ministral/native/predictor_shared_input.cu:16-41) bit for bit against the oracle on
the layer's own y, the flags carrying the enqueue's epoch and the bell counting launches;
batch rows each normalized on their own, the flags released once per launch. A fused launch
runs it in its own last workgroup (batch 1 and 4); the split entry point and a dense (batch 32,
matrix-core) launch run it as a kernel after the layer."""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.backend import Mapped
from leanstream_amd.workload import DeviceLayer

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


# fused launches run the epilogue in their last workgroup; the split entry point (candidate 4)
# and the dense path (batch 32) launch epilogue_kernel after the layer
@pytest.mark.parametrize("key,table", [("c2", None), ("c2", [[4]]), ("c1b4", None), ("c1d32", None)],
                         ids=["c2-fused", "c2-split", "c1b4-fused", "c1d32-dense"])
def test_epilogue_publishes_hidden_and_rmsnorm(torch_gpu, key, table):
    torch = torch_gpu
    cfg = synth.CONFIGS[key]
    log(f"case: epilogue {cfg.name} table {table}")
    layer = DeviceLayer(cfg, offline_table=table) if table else DeviceLayer(cfg)
    d, rows = cfg.width, cfg.batch
    rng = np.random.default_rng(17)
    residual_h = rng.standard_normal(rows * d).astype(np.float16)
    weight_h = rng.uniform(0.5, 1.5, d).astype(np.float16)
    residual = torch.from_numpy(residual_h).cuda()
    weight = torch.from_numpy(weight_h).cuda()
    hidden = torch.empty(rows * d, dtype=torch.float16, device="cuda")
    normed = torch.empty(rows * d, dtype=torch.float16, device="cuda")
    flags = Mapped(3, np.uint32)            # hidden flag, norm flag, bell (host-coherent)
    flags.host[:] = 0
    eps = 1e-5
    layer.backend.set_epilogue(residual, hidden, flags.ptr, weight, normed, flags.ptr + 4, flags.ptr + 8, eps)
    layer.seal_empty_queue(7)
    for launch, epoch in enumerate((7, 8)):
        if launch:
            layer.seal_empty_queue(epoch)
        layer.run_core(epoch=epoch)
        torch.cuda.synchronize()
        assert layer.backend.status() == 0
        if table:
            assert layer.backend.last_candidate() == table[0][0]
        assert flags.host.tolist() == [epoch, epoch, launch + 1]
        y = layer.y.cpu().numpy()
        want_hidden = oracle.publish_hidden(residual_h, y)
        assert np.array_equal(hidden.cpu().numpy().view(np.uint16), want_hidden.view(np.uint16))
        got = normed.cpu().numpy().reshape(rows, d)
        for b in range(rows):
            want = oracle.rmsnorm(want_hidden[b * d:(b + 1) * d], weight_h, eps)
            assert np.array_equal(got[b].view(np.uint16), want.view(np.uint16)), f"row {b}"
    # without the epilogue the layer output is unchanged and nothing is published
    y_with = layer.y.clone()
    layer.backend.set_epilogue(None, None)
    layer.seal_empty_queue(9)
    layer.run_core(epoch=9)
    torch.cuda.synchronize()
    assert torch.equal(layer.y, y_with)
    assert flags.host.tolist() == [8, 8, 2]
    layer.close()
    flags.close()
