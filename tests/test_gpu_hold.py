"""ls_hold_stream, the benchmark's stream hold: work queued behind it waits until the host
releases the flag, and the hold ends by itself once its bound passes."""
import time

import numpy as np
import pytest

from leanstream_amd import _native
from leanstream_amd.backend import Mapped

pytestmark = pytest.mark.gpu


def test_hold_waits_for_release_then_for_its_bound(torch_gpu):
    torch = torch_gpu
    lib = _native.library()
    stream = torch.cuda.current_stream()
    flag = Mapped(1, np.uint32)
    dst = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    try:
        print("case: hold released by the host", flush=True)
        flag.host[0] = 0
        torch.cuda.synchronize()
        assert lib.ls_hold_stream(stream.cuda_stream, flag.ptr, 200_000_000) == 0   # 2 s bound
        assert lib.ls_synth_bytes(dst.data_ptr(), dst.numel(), 7, stream.cuda_stream) == 0
        done = torch.cuda.Event()
        done.record(stream)
        time.sleep(0.05)
        assert not done.query(), "work behind the hold ran before the release"
        flag.release(0, 1)
        done.synchronize()
        assert int(dst.sum()) > 0
        print("case: hold ends at its bound", flush=True)
        flag.host[0] = 0
        t0 = time.monotonic()
        assert lib.ls_hold_stream(stream.cuda_stream, flag.ptr, 2_000_000) == 0   # 20 ms, never released
        torch.cuda.synchronize()
        assert time.monotonic() - t0 < 2.0
        assert lib.ls_hold_stream(stream.cuda_stream, None, 1) != 0
        assert lib.ls_hold_stream(stream.cuda_stream, flag.ptr, 0) != 0
    finally:
        torch.cuda.synchronize()
        flag.close()
