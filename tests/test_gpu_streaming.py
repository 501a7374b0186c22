"""Streaming decode over host-staged layers on the GPU (HostStagingIO + HipCopyEngine +
Runtime/LayerStep + the persistent consumer).

Each layer's ranked groups are copied from pinned host memory into the staging arena
as they arrive (seeded exponential arrival gaps) and published READY to the kernel that
was pre-enqueued for the layer. Checks: the output of every layer against the oracle
(relative L2 <= 1e-3, max-abs <= 2e-2 on fp16 y, which adds at most half an fp16 ulp to
the fp32 bound), bit-identity with the same layer run from HBM-resident groups (the
reduction does not depend on readiness order), the final queue state and descriptors
(bit-exact), exactly-once execution, and the transport's per-group stamps.
"""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth
from leanstream_amd.streaming import COPY_HIP, TIME_FIELDS, StreamingDecode
from leanstream_amd.workload import DeviceLayer

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-2


def log(msg):
    print(msg, flush=True)


def compare(y, ref, what):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = float(np.abs(y - ref).max())
    log(f"{what}: rel_l2={rel:.3e} max_abs={mx:.3e}")
    assert rel <= REL_L2 and mx <= MAX_ABS, (rel, mx)


def test_streamed_layers_match_oracle(torch_gpu):
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    layers = 4
    log(f"case: streamed decode {sc.name} layers={layers} arrivals on")
    sd = StreamingDecode(sc, layers=layers)
    try:
        times, stamps = sd.run()
        torch.cuda.synchronize()
        assert sd.backend.status() == 0
        log("layer us: " + ", ".join(f"{(t[6] - t[0]) / 1e3:.1f}" for t in times))
        ys = sd.y.cpu().numpy()
        k, n = sd.cfg.active, sd.cfg.groups
        for l in range(layers):
            hl = sd.host_layer(l)
            rows = synth.descriptors(hl.cfg, sd.ranks[l])
            ref = oracle.layer(rows, k, hl.cache, hl.scales, hl.x, sd.cfg.width, sd.cfg.group_size, threads=8)
            compare(ys[l], ref["y32"], f"layer {l}")
            # transport: every ranked group admitted, copied no earlier than it arrived, completed
            st = stamps[l]
            ranked = sd.ranks[l]
            assert np.all(st[ranked] > 0)
            assert np.all(st[ranked, 1] >= sd.arrivals[l][ranked])
            others = np.setdiff1d(np.arange(n), ranked)
            assert np.all(st[others] == 0)
        # every destination computed exactly once per layer
        assert np.all(sd.executions.cpu().numpy() == layers)
        # queue of the last layer: descriptors in final order, all published once
        desc, idx, ctrl = sd.queue()
        l = layers - 1
        want = np.zeros((k, 5), dtype=np.uint32)
        want[:, 0] = sd.ranks[l]
        want[:, 1] = l * n + synth.physical_of(sd.ranks[l], n)
        want[:, 2] = sd.ranks[l]            # staging slot = logical group
        want[:, 3] = np.arange(k)
        want[:, 4] = 1                       # SourceKind::Staging
        assert np.array_equal(desc[:k], want)
        assert ctrl[0] == k and ctrl[2] == k and ctrl[5] == 0
        assert sorted(idx[:k].tolist()) == list(range(k))
        # times are monotone within each layer
        assert np.all(np.diff(times.astype(np.int64), axis=1) >= 0), dict(zip(TIME_FIELDS, times[0]))
    finally:
        sd.close()


def test_streamed_layer_bit_identical_to_resident_layer(torch_gpu):
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    log(f"case: streamed vs resident {sc.name} layers 0..1")
    sd = StreamingDecode(sc, layers=2)
    try:
        sd.run()
        torch.cuda.synchronize()
        streamed = sd.y.cpu().numpy().copy()
        for l in range(2):
            lc = sc.layer_config(l)
            layer = DeviceLayer(lc, logical=sd.ranks[l])
            try:
                layer.x.copy_(sd.x)
                layer.seal_empty_queue(1)
                layer.run_core(epoch=1)
                torch.cuda.synchronize()
                assert layer.backend.status() == 0
                resident = layer.y.cpu().numpy()
                assert np.array_equal(resident.view(np.uint16), streamed[l].view(np.uint16)), f"layer {l}"
            finally:
                layer.close()
        # a second pass over the same layers: same bits (staging slots are rewritten)
        sd.run()
        torch.cuda.synchronize()
        assert np.array_equal(sd.y.cpu().numpy().view(np.uint16), streamed.view(np.uint16))
    finally:
        sd.close()


def test_streamed_layers_without_arrival_delay(torch_gpu):
    """Copies issued as soon as admitted, through hipMemcpyAsync instead of direct SDMA,
    or cut into pieces over 16 SDMA engines: same outputs as with delays."""
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    log(f"case: streamed decode {sc.name} layers=3 no arrival delay: hipMemcpyAsync on 1 stream with qd 4; "
        f"24 KB SDMA pieces on 16 engines")
    a = StreamingDecode(sc, layers=3)
    b = StreamingDecode(sc, layers=3, arrivals=False, qd=4, copy_engine=COPY_HIP, copy_queues=1)
    c = StreamingDecode(sc, layers=3, arrivals=False, copy_queues=16, copy_chunk=24576)   # 4 pieces per group
    try:
        a.run()
        b.run()
        c.run()
        torch.cuda.synchronize()
        want = a.y.cpu().numpy().view(np.uint16)
        assert np.array_equal(want, b.y.cpu().numpy().view(np.uint16))
        assert np.array_equal(want, c.y.cpu().numpy().view(np.uint16))
    finally:
        a.close()
        b.close()
        c.close()


def test_full_decode_step_matches_oracle(torch_gpu):
    """The whole streaming decode step of the C3 shape: 36 host-staged layers, every one
    against the oracle, every destination executed once per layer."""
    torch = torch_gpu
    sc = synth.STREAMS["c3"]
    layers = sc.layers
    log(f"case: full streamed decode step {sc.name} layers={layers} arrivals on")
    sd = StreamingDecode(sc, layers=layers)
    try:
        sd.run()
        torch.cuda.synchronize()
        assert sd.backend.status() == 0
        ys = sd.y.cpu().numpy()
        k = sd.cfg.active
        worst = 0.0
        for l in range(layers):
            hl = sd.host_layer(l)
            rows = synth.descriptors(hl.cfg, sd.ranks[l])
            ref = oracle.layer(rows, k, hl.cache, hl.scales, hl.x, sd.cfg.width, sd.cfg.group_size, threads=8)
            y = ys[l].astype(np.float64)
            r = ref["y32"].astype(np.float64)
            rel = np.linalg.norm(y - r) / max(np.linalg.norm(r), 1e-30)
            mx = float(np.abs(y - r).max())
            assert rel <= REL_L2 and mx <= MAX_ABS, (l, rel, mx)
            worst = max(worst, rel)
        log(f"  {layers} layers within tolerance, worst rel_l2 {worst:.3e}")
        assert np.all(sd.executions.cpu().numpy() == layers)
    finally:
        sd.close()
