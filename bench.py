#!/usr/bin/env python3
"""Benchmark: microseconds per sparse INT4 MLP layer and achieved HBM bandwidth on one MI355X.

Workload (one GPU, batch 1): Ministral-8B-shaped sparse MLP layer, d_model 4096,
d_ffn 12288 = 192 groups of 64 neurons, 58 active groups (30%, seeded ranking), INT4 g128
weights with fp16 scales U(0.005, 0.02), fp16 x ~ N(0, 1), all weights HBM-resident and
every group ready before launch (resident core descriptors).

A "step" is one enqueue of the layer (fused persistent kernel: gate/up, SiLU, down
projection, compact reduction). Steps rotate over independent copies of the layer whose
active bytes total more than the 256 MB Infinity Cache, so every step reads HBM.

Printed: one JSON line (rank 0). value = microseconds per layer in the back-to-back
pipeline (HIP events on the launch stream around the timed steps, divided by steps; the
first steps are queued behind a bounded hold of the stream before the region starts, so
the host's submission latency is not inside it: timed_steps).
roofline.achieved = algorithmic bytes per layer / that per-layer time.

The default run also times the layer stack of a decode step as one launch per step (36
distinct C2 layers, and 36 of C1, chained through the epilogue: "pipelined"), and every
other workload of the path with fewer steps (C1, C4 at batch 1 and 4, the Group2
Ministral-3 shape, C5 dense batch 32, and a few C3 decode steps: "secondary"), in the same
JSON line.

--workload c3 instead measures a streaming decode step: 36 layers of the d_model 1024
shape whose 16 active groups per layer are staged from pinned host memory by SDMA
copies as they arrive (exponential gaps of mean 5 us in rank order), each published
READY to the layer's pre-enqueued persistent consumer; value = wall microseconds per
layer, with the I/O floor (last arrival), copy latency and completion tail beside it.
"""
import argparse
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "µs per sparse INT4 MLP layer + achieved HBM GB/s (% roofline), batch 1, 8B shape"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 * 2 ** 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 400 layers; 20 decode steps for c3)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 50 layers; 2 decode steps for c3)")
    ap.add_argument("--workload", default="c2", choices=["c1", "c2", "c4", "c4b4", "c5", "c1d32", "c3", "g2",
                                                          "chain", "c1chain"],
                    help="c3: 36-layer streaming decode step staged from pinned host memory; chain / c1chain: "
                         "36 distinct C2 / C1 layers chained through the epilogue in one launch")
    ap.add_argument("--layers", type=int, default=36, help="layers per chain launch (chain workloads)")
    ap.add_argument("--stamps", default=None, help="chain workloads: write per-layer phase stamps (.npy) here")
    ap.add_argument("--candidate", type=int, default=None, help="force a kernel candidate id (offline LUT of one entry)")
    ap.add_argument("--copies", type=int, default=0, help="layer copies to rotate over (0: enough to exceed 256 MB)")
    ap.add_argument("--isolated", type=int, default=100, help="isolated launches timed one by one")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="default c2 run only: skip the shorter back-to-back runs of the other workloads")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 plain 64 MiB device copies (counter calibration for rocprofv3 --pmc)")
    return ap.parse_args()


def copy_calibration():
    """Five plain device-to-device copies of 64 MiB: each dispatch reads and writes exactly
    67108864 bytes, the known size that FETCH_SIZE / WRITE_SIZE are scaled against."""
    import torch

    n = 64 * 2 ** 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "dispatches": 5}), flush=True)


def percentile(v, q):
    v = sorted(v)
    if not v:
        return None
    k = (len(v) - 1) * q
    lo, hi = math.floor(k), math.ceil(k)
    return v[lo] + (v[hi] - v[lo]) * (k - lo)


def traffic_from_profiles(workload_name):
    """HBM bytes per launch measured with rocprofv3 PMC counters (committed summary)."""
    f = ROOT / "profiles" / f"traffic_{workload_name}.txt"
    if not f.is_file():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


def host_cpu():
    """(logical CPUs of the host, CPU model string)."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return os.cpu_count() or 1, model


# A one-GPU job gets a share of 16 host CPUs (OMP_NUM_THREADS is set to it): the
# baseline's thread pool stays within that share whatever the host's CPU count.
CPU_SHARE = 16


def cpu_baseline(cfg, budget_s):
    """The oracle (CPU restatement of the reference arithmetic) timed on the host cores."""
    import numpy as np

    if not (ROOT / "oracle" / "liboracle.so").is_file():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    import oracle
    from leanstream_amd import synth

    hl = synth.host_layer(cfg)
    rows = synth.descriptors(cfg, synth.active_groups(cfg))
    host_cpus, model = host_cpu()
    share = int(os.environ.get("OMP_NUM_THREADS", CPU_SHARE) or CPU_SHARE)
    threads = max(1, min(share, host_cpus))
    out = {}
    for label, nthreads, share in (("all", threads, 0.7), ("one", 1, 0.3)):
        t_end = time.perf_counter() + budget_s * share
        n = 0
        t0 = time.perf_counter()
        while True:
            oracle.layer(rows, len(rows), hl.cache, hl.scales, hl.x, cfg.width, cfg.group_size, threads=nthreads)
            n += 1
            if time.perf_counter() >= t_end:
                break
        out[label] = ((time.perf_counter() - t0) / n * 1e6, n, nthreads)
    us_all, n_all, t_all = out["all"]
    us_one, n_one, _ = out["one"]
    return {
        "value": round(us_all, 1),
        "unit": "us/layer",
        "cores": t_all,
        "kind": "port",
        "sample": f"{n_all} full layers ({cfg.name}) with {t_all} OpenMP threads (the job's CPU share of a "
                  f"{host_cpus}-CPU host); single thread: {us_one:.0f} us/layer over {n_one} layers",
        "gbs": round(cfg.algorithmic_bytes() / us_all / 1e3, 2),
        "single_thread_us": round(us_one, 1),
        "host_cpus": host_cpus,
        "cpu_model": model,
    }


def control_plane_timing(groups=64, active=16, seconds=2.0):
    """The C1 layer's control plane on one host thread (leanstream_amd/control_plane_timing:
    Runtime/LayerStep, WeightManager, ExecutionQueue; begin, prediction update, enqueue,
    finalize, READY publication of every active group, commit), µs per layer."""
    exe = ROOT / "leanstream_amd" / "control_plane_timing"
    if not exe.is_file():
        subprocess.run(["make", "-s", "-C", str(ROOT / "leanstream_amd" / "csrc")], check=True)
    out = subprocess.run([str(exe), str(groups), str(active), str(seconds)], check=True, capture_output=True,
                         text=True, timeout=60 + seconds).stdout
    r = json.loads(out.strip().splitlines()[-1])
    r["what"] = ("Runtime::begin_layer + update_prediction + enqueue_compute (no launch) + finalize + READY "
                 "publication of every active group + commit, host memory, one thread")
    return r


def decode_steps(sc, steps, warmup, **kw):
    """`steps` timed decode steps of the streaming shape `sc` (after `warmup` untimed ones):
    (arrival schedule, wall seconds per step, per-layer host times, per-group stamps)."""
    import numpy as np
    import torch

    from leanstream_amd.streaming import StreamingDecode

    sd = StreamingDecode(sc, **kw)
    try:
        for _ in range(warmup):
            sd.run()
        torch.cuda.synchronize()
        walls, times, stamps = [], [], []
        for _ in range(steps):
            t0 = time.perf_counter()
            t, st = sd.run()
            walls.append(time.perf_counter() - t0)
            times.append(t)
            stamps.append(st)
        assert sd.backend.status() == 0, sd.backend.status()
        return sd.arrivals.copy(), np.array(walls), np.concatenate(times), np.concatenate(stamps)
    finally:
        sd.close()


def timed_steps(stream, submit, steps, queued=64):
    """Milliseconds of `steps` calls of submit(i) back to back on `stream`, from HIP events on
    the stream around them. The GPU is idle when this starts; the stream is held by a bounded
    one-wave kernel (ls_hold_stream) while the start event and the first `queued` steps are
    queued behind it, then released: the region holds exactly the steps, back to back,
    without the host's submission latency before the first (the later ones are submitted
    while the queued ones run)."""
    import numpy as np
    import torch

    from leanstream_amd import _native
    from leanstream_amd.backend import Mapped

    lib = _native.library()
    flag = Mapped(1, np.uint32)
    try:
        flag.host[0] = 0
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        rc = lib.ls_hold_stream(stream.cuda_stream, flag.ptr, 100_000_000)   # released well within 1 s
        if rc:
            raise RuntimeError(f"ls_hold_stream failed: {rc}")
        start.record(stream)
        first = min(steps, queued)
        for i in range(first):
            submit(i)
        flag.release(0, 1)
        for i in range(first, steps):
            submit(i)
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop)
    finally:
        flag.close()


def timed_layer(cfg, steps, warmup, copies=0, table=None, isolated=0):
    """One layer shape, every group resident and ready before launch: microseconds per layer
    back to back (HIP events on the launch stream around `steps` launches that rotate over
    `copies` copies of the layer, by default enough to exceed the Infinity Cache), then
    `isolated` launches timed one by one on an otherwise idle GPU."""
    import torch

    from leanstream_amd.workload import DeviceLayer

    active_bytes = cfg.active * cfg.group_bytes + cfg.active * cfg.scale_words * 2
    copies = copies or max(2, math.ceil(1.5 * MALL_BYTES / active_bytes))
    print(f"[bench] workload {cfg.name}: k={cfg.active} B_alg={cfg.algorithmic_bytes()} copies={copies}",
          file=sys.stderr, flush=True)
    layer = DeviceLayer(cfg, copies=copies, with_y32=False, diagnostics=False, offline_table=table)
    try:
        layer.seal_empty_queue(1)
        stream = torch.cuda.current_stream()
        for i in range(warmup):
            layer.run_core(copy=i % copies, epoch=1)
        torch.cuda.synchronize()
        assert layer.backend.status() == 0, f"device status {layer.backend.status()}"
        print(f"[bench] warmup done, timing {steps} steps", file=sys.stderr, flush=True)
        # back-to-back pipeline: events on the launch stream around the timed steps
        ms_total = timed_steps(stream, lambda i: layer.run_core(copy=i % copies, epoch=1), steps)
        # isolated layers: one event pair per launch, idle GPU between launches
        iso = []
        for i in range(isolated):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            layer.run_core(copy=i % copies, epoch=1)
            e1.record(stream)
            e1.synchronize()
            iso.append(e0.elapsed_time(e1) * 1000.0)
        status = layer.backend.status()
        candidate = layer.backend.last_candidate()
        workers = layer.backend.max_workers
    finally:
        layer.close()
    assert status == 0, f"device status {status}"
    return {"us": ms_total * 1000.0 / steps, "ms_total": ms_total, "iso": iso, "copies": copies,
            "active_bytes": active_bytes, "candidate": candidate, "workers": workers}


def timed_chain(cfg, steps, warmup, layers=36, isolated=0, stamps=False):
    """A decode step's MLP stack: `layers` distinct layers of one shape chained through the
    epilogue (layer i's hidden state fp16(residual_i + y_i) is layer i + 1's residual, and its
    RMSNorm times the layer's weight is layer i + 1's input), computed by one persistent
    launch (ls_hip_enqueue_chain). `steps` launches back to back, HIP events on the launch
    stream around them; microseconds per layer = elapsed / (steps * layers)."""
    import torch

    from leanstream_amd.workload import DeviceLayer

    print(f"[bench] chain {cfg.name}: {layers} distinct layers per launch, B_alg/layer={cfg.algorithmic_bytes()}",
          file=sys.stderr, flush=True)
    layer = DeviceLayer(cfg, copies=layers, with_y32=False, diagnostics=False)
    out = {}
    try:
        outputs = layer.chain_outputs(layers)
        norm = layer.chain_norm_weights(layers)
        blocks = layer.backend.chain_blocks(layer.chain_layers(list(range(layers)), outputs, output32=False,
                                                               norm=norm))
        stream = torch.cuda.current_stream()
        sid = stream.cuda_stream
        for _ in range(warmup):
            layer.backend.enqueue_chain(blocks, sid)
        torch.cuda.synchronize()
        assert layer.backend.status() == 0, f"device status {layer.backend.status()}"
        print(f"[bench] chain warmup done, timing {steps} launches", file=sys.stderr, flush=True)
        ms_total = timed_steps(stream, lambda i: layer.backend.enqueue_chain(blocks, sid), steps, queued=8)
        iso = []
        for _ in range(isolated):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            layer.backend.enqueue_chain(blocks, sid)
            e1.record(stream)
            e1.synchronize()
            iso.append(e0.elapsed_time(e1) * 1000.0)
        if stamps:
            w = layer.backend.chain_workers + 1
            st = torch.zeros(layers * w * 4 * 32, dtype=torch.int64, device="cuda")
            layer.backend.set_chain_stamps(st, layers)
            layer.backend.enqueue_chain(blocks, sid)
            torch.cuda.synchronize()
            out["stamps"] = st.cpu().numpy().reshape(layers, w * 4, 32)
            layer.backend.set_chain_stamps(None, 0)
        status = layer.backend.status()
        out["workers"] = layer.backend.chain_workers
    finally:
        layer.close()
    assert status == 0, f"device status {status}"
    out.update({"us": ms_total * 1000.0 / (steps * layers), "ms_total": ms_total, "iso": iso, "layers": layers})
    return out


def timed_dependent(cfg, steps, warmup, layers=36):
    """The same decode-step stack as timed_chain, one launch per layer: layer i's enqueue (x =
    layer i - 1's RMSNorm output) followed by its epilogue (hidden state and RMSNorm times layer
    i + 1's weight, the next layer's input), in stream order, so each layer waits for the one
    before it -- the per-launch path with the decode step's dependency. µs per layer."""
    import torch

    from leanstream_amd.backend import MODE_PROGRESSIVE
    from leanstream_amd.workload import DeviceLayer

    print(f"[bench] dependent per-launch stack {cfg.name}: {layers} layers", file=sys.stderr, flush=True)
    layer = DeviceLayer(cfg, copies=layers, with_y32=False, diagnostics=False)
    try:
        d = cfg.width
        norm = layer.chain_norm_weights(layers + 1)
        xs = torch.empty(layers + 1, d, dtype=torch.float16, device="cuda")
        xs[0].copy_(layer.x)
        hidden = torch.empty(layers + 1, d, dtype=torch.float16, device="cuda")
        hidden[0].copy_(layer.x)
        ys = torch.empty(layers, d, dtype=torch.float16, device="cuda")
        layer.seal_empty_queue(1)
        stream = torch.cuda.current_stream()
        sid = stream.cuda_stream
        be = layer.backend

        def step(_):
            for i in range(layers):
                be.set_epilogue(hidden[i], hidden[i + 1], norm_weight=norm[i + 1], norm_output=xs[i + 1], eps=1e-5)
                be.enqueue(0, 0, 1, xs[i], ys[i], sid, layer.core_ptr(i), layer.k, layer.queue, MODE_PROGRESSIVE)

        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        ms_total = timed_steps(stream, step, steps, queued=steps)
        be.set_epilogue(None, None)
        status = be.status()
    finally:
        layer.close()
    assert status == 0, f"device status {status}"
    return {"us": ms_total * 1000.0 / (steps * layers), "ms_total": ms_total}


# Shorter back-to-back runs of the other workloads, in the default run's JSON line:
# (key, timed steps, warm-up steps); c3 in decode steps of 36 layers.
SECONDARY = (("c1", 200, 20), ("c4", 200, 20), ("c4b4", 100, 10), ("g2", 200, 20), ("c5", 100, 10), ("c3", 5, 1))


def secondary_workloads():
    """Every other workload of the path, measured as its own bench line would (fewer steps).
    A workload that fails is reported with its error; the headline and the others stand."""
    from leanstream_amd import synth

    out = {}
    for key, steps, warmup in SECONDARY:
        try:
            if key == "c3":
                sc = synth.STREAMS["c3"]
                print(f"[bench] streaming {sc.name}: {sc.layers} layers x {steps} steps", file=sys.stderr,
                      flush=True)
                _, walls, _, _ = decode_steps(sc, steps, warmup)
                out[key] = {"workload": sc.name, "us_per_layer": round(float(walls.mean()) * 1e6 / sc.layers, 2),
                            "steps": steps, "kind": "host-staged decode step, wall clock"}
                continue
            cfg = synth.CONFIGS[key]
            r = timed_layer(cfg, steps, warmup)
            gbs = cfg.algorithmic_bytes() / r["us"] / 1e3
            out[key] = {"workload": cfg.name, "us_per_layer": round(r["us"], 3), "steps": steps,
                        "algorithmic_bytes": cfg.algorithmic_bytes(), "achieved_GBps": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4)}
        except Exception as exc:  # noqa: BLE001 -- reported in the line, not fatal to it
            print(f"[bench] {key} failed: {exc!r}", file=sys.stderr, flush=True)
            out[key] = {"error": repr(exc)[:300]}
    return out


def pipelined_workloads():
    """The decode step's layer stack in one launch per step (ls_hip_enqueue_chain): 36 distinct
    C2 layers and 36 distinct C1 layers chained through the epilogue (hidden state as the next
    residual, its RMSNorm as the next input), microseconds per layer of back-to-back launches;
    beside it the same stack launched layer by layer with the epilogue between layers."""
    from leanstream_amd import synth

    out = {}
    for key, layers in (("c2", 36), ("c1", 36)):
        cfg = synth.CONFIGS[key]
        try:
            r = timed_chain(cfg, 20, 3, layers=layers)
            gbs = cfg.algorithmic_bytes() / r["us"] / 1e3
            out[key] = {"workload": f"chain{layers}_{cfg.name}", "layers_per_launch": layers,
                        "us_per_layer": round(r["us"], 3), "steps": 20, "achieved_GBps": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4)}
            dep = timed_dependent(cfg, 5, 1, layers=layers)
            out[key]["per_launch_dependent_us_per_layer"] = round(dep["us"], 3)
        except Exception as exc:  # noqa: BLE001 -- reported in the line, not fatal to it
            print(f"[bench] chain {key} failed: {exc!r}", file=sys.stderr, flush=True)
            out[key] = {"error": repr(exc)[:300]}
    return out


def streaming_bench(a):
    """C3: decode steps of 36 host-staged layers (HostStagingIO + SDMA copies + Runtime/LayerStep
    + the persistent consumer). A step's time is host wall clock around ls_stream_run (the
    call returns after the last layer's completion word and commit)."""
    import numpy as np

    from leanstream_amd import synth

    sc = synth.STREAMS["c3"]
    steps, warmup = a.steps or 20, 2 if a.warmup is None else a.warmup
    print(f"[bench] streaming {sc.name}: {sc.layers} layers x {steps} steps", file=sys.stderr, flush=True)

    def run(**kw):
        return decode_steps(sc, steps, warmup, **kw)

    arrivals, walls, times, stamps = run()
    us_layer = walls.mean() * 1e6 / sc.layers
    layer_us = (times[:, 6] - times[:, 0]) / 1e3
    last_arrival = np.tile(arrivals.max(axis=1), steps) / 1e3
    last_ready = stamps[:, :, 2].max(axis=1) / 1e3
    complete = (times[:, 5] - times[:, 0]) / 1e3
    sub, done = stamps[:, :, 1].astype(np.int64), stamps[:, :, 2].astype(np.int64)
    lat = (done - sub)[sub > 0] / 1e3
    print(f"[bench] delayed arrivals: {us_layer:.1f} us/layer", file=sys.stderr, flush=True)
    # the same layers with every copy issued at admission: the PCIe/SDMA-bound rate
    _, walls0, times0, stamps0 = run(arrivals=False, copy_queues=16)
    us0 = walls0.mean() * 1e6 / sc.layers
    staged = sc.layer.active * sc.layer.group_bytes
    print(f"[bench] no arrival delay: {us0:.1f} us/layer", file=sys.stderr, flush=True)
    # one layer of the shape with its groups resident in HBM (all ready before launch)
    resident_us = timed_layer(sc.layer_config(0), 200, 20, copies=1)["us"]
    result = {
        "metric": "µs per host-staged sparse INT4 MLP layer (streaming decode step of 36 layers), batch 1",
        "value": round(us_layer, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(walls.mean() * 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16-f32acc",
        "data": "synthetic (seeded INT4 weights per layer in pinned host memory, N(0,1) group scores per layer, "
                "exponential arrival gaps of mean 5 us in rank order)",
        "config": {
            "workload": sc.name,
            "layers": sc.layers,
            "d_model": sc.layer.width,
            "d_ffn": sc.layer.ffn,
            "active_groups": sc.layer.active,
            "staged_bytes_per_layer": staged,
            "arrival_gap_mean_us": sc.arrival_mean_ns / 1e3,
            "copy_engine": "sdma",
            "copy_queues": 8,
            "qd": 24,
        },
        "io": {
            "last_arrival_us": round(float(last_arrival.mean()), 2),
            "last_ready_us": round(float(last_ready.mean()), 2),
            "complete_us": round(float(complete.mean()), 2),
            "layer_wall_us_p50": round(float(np.median(layer_us)), 2),
            "after_last_arrival_us": round(float(us_layer - last_arrival.mean()), 2),
            "copy_latency_us_p50_p90": [round(float(np.percentile(lat, 50)), 2), round(float(np.percentile(lat, 90)), 2)],
            "kernel_done_after_last_ready_us": round(float((complete - last_ready).mean()), 2),
        },
        "no_arrival_delay": {
            "us_per_layer": round(us0, 2),
            "h2d_GBps": round(staged / us0 / 1e3, 2),
            "copy_queues": 16,
        },
        "resident_layer_us": round(resident_us, 3),
    }
    if not a.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(sc.layer_config(0), a.cpu_seconds)
        except Exception as exc:
            result["cpu_baseline"] = {"value": None, "error": str(exc)}
    print(json.dumps(result), flush=True)


def chain_bench(a):
    from leanstream_amd import synth

    cfg = synth.CONFIGS["c2" if a.workload == "chain" else "c1"]
    steps = 20 if a.steps is None else a.steps
    warmup = 3 if a.warmup is None else a.warmup
    r = timed_chain(cfg, steps, warmup, layers=a.layers, isolated=min(a.isolated, 20), stamps=bool(a.stamps))
    if a.stamps:
        import numpy as np

        np.save(a.stamps, r["stamps"])
    balg = cfg.algorithmic_bytes()
    achieved = balg / r["us"] / 1e3
    result = {
        "metric": METRIC,
        "value": round(r["us"], 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(r["ms_total"] / steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16-f32acc",
        "data": "synthetic (seeded splitmix64 INT4 weights per layer, U(lo,hi) fp16 scales, N(0,1) fp16 x)",
        "config": {
            "workload": f"chain{a.layers}_{cfg.name}",
            "layers_per_launch": a.layers,
            "d_model": cfg.width,
            "d_ffn": cfg.ffn,
            "group_size": cfg.group_size,
            "active_groups": cfg.active,
            "batch": cfg.batch,
            "algorithmic_bytes_per_layer": balg,
            "chain_workers": r["workers"],
            "isolated_launch_us_p50": round(percentile(r["iso"], 0.5), 2) if r["iso"] else None,
        },
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
    }
    print(json.dumps(result), flush=True)


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "the path runs on one GPU; --gpus must be 1 (multi-GPU sharding is design-only)"}))
        sys.exit(2)
    if a.copy_calibration:
        copy_calibration()
        return
    if a.workload == "c3":
        streaming_bench(a)
        return
    if a.workload in ("chain", "c1chain"):
        chain_bench(a)
        return
    a.steps = 400 if a.steps is None else a.steps
    a.warmup = 50 if a.warmup is None else a.warmup
    from leanstream_amd import synth

    cfg = synth.CONFIGS[a.workload]
    table = None if a.candidate is None else [[a.candidate]]
    r = timed_layer(cfg, a.steps, a.warmup, copies=a.copies, table=table, isolated=a.isolated)
    us_per_layer, ms_total, iso = r["us"], r["ms_total"], r["iso"]
    copies, active_bytes, candidate, workers = r["copies"], r["active_bytes"], r["candidate"], r["workers"]

    balg = cfg.algorithmic_bytes()
    achieved = balg / us_per_layer / 1e3  # GB/s
    traffic = traffic_from_profiles(cfg.name)
    result = {
        "metric": METRIC,
        "value": round(us_per_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_total / a.steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16-f32acc",
        "data": "synthetic (seeded splitmix64 INT4 weights, U(lo,hi) fp16 scales, N(0,1) fp16 x)",
        "config": {
            "workload": cfg.name,
            "d_model": cfg.width,
            "d_ffn": cfg.ffn,
            "group_size": cfg.group_size,
            "active_groups": cfg.active,
            "batch": cfg.batch,
            "algorithmic_bytes": balg,
            "rotation_copies": copies,
            "rotation_active_bytes": copies * active_bytes,
            "candidate": candidate,
            "resident_workers": workers,
            "isolated_us_p10_p50_p90": [round(percentile(iso, q), 3) for q in (0.1, 0.5, 0.9)] if iso else None,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
    }
    if a.workload == "c2" and a.candidate is None and not a.copies and not a.no_secondary:
        result["pipelined"] = pipelined_workloads()
        result["secondary"] = secondary_workloads()
    if not a.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(cfg, a.cpu_seconds)
        except Exception as exc:  # the GPU figure stands on its own
            result["cpu_baseline"] = {"value": None, "error": str(exc)}
        if a.workload == "c2":
            try:
                result["cpu_baseline"]["control_plane_c1"] = control_plane_timing()
            except Exception as exc:  # noqa: BLE001 -- reported, not fatal
                result["cpu_baseline"]["control_plane_c1"] = {"error": repr(exc)[:300]}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
