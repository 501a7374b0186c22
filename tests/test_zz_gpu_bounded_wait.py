"""Every device wait is bounded: a layer whose epoch is never published ends with the
timeout status bit instead of hanging (the condition is forced from the host with a
short spin limit on the kernel's own bounded wait)."""
import time

import numpy as np
import pytest

from leanstream_amd import synth
from leanstream_amd.backend import MODE_PROGRESSIVE, STATUS_TIMEOUT
from leanstream_amd.workload import DeviceLayer

pytestmark = pytest.mark.gpu


def test_unpublished_epoch_times_out(torch_gpu):
    torch = torch_gpu
    print("case: epoch never published, spin limit 20 ms", flush=True)
    cfg = synth.CONFIGS["c1"]
    layer = DeviceLayer(cfg)
    layer.backend.set_spin_limit(2_000_000)   # 20 ms of the 100 MHz device clock
    q = layer.queue
    q.write_descriptors(synth.descriptors(cfg, layer.logical))
    q.reset(7)   # epoch word stays 0: the consumer never sees epoch 7
    t0 = time.time()
    layer.backend.enqueue(0, 0, 7, layer.x, layer.y, torch.cuda.current_stream().cuda_stream, None, 0, q,
                          MODE_PROGRESSIVE)
    torch.cuda.synchronize()
    assert time.time() - t0 < 5.0
    assert layer.backend.status() & STATUS_TIMEOUT
    layer.backend.clear_status()
    layer.backend.set_spin_limit(200_000_000)
    # the backend keeps working afterwards
    layer.seal_empty_queue(8)
    layer.run_core(epoch=8)
    torch.cuda.synchronize()
    assert layer.backend.status() == 0
    assert np.isfinite(layer.y32.cpu().numpy()).all()
    layer.close()
