"""Per-wave phase timeline of one persistent layer launch, from the kernels' own stamps.

With a stamps buffer bound (HipLayerBuffers::stamps), every wave of the fused kernel writes
the device's 100 MHz clock (s_memrealtime) at fixed points of its walk (lsamd::StampPhase in
leanstream_amd/csrc/mlp_args.h). This diagnostic runs a workload's layer back to back over
rotated copies, then stamps one launch after each batch of warm launches, and prints each
phase's time after the first wave's start (percentiles over waves and repetitions), plus
per-wave intervals of the waves that hold a down item.

    python -m leanstream_amd.phase_stamps --workload c2
"""
import argparse

import numpy as np

from . import synth

PHASES = {0: "entry", 1: "descriptors in", 5: "item 0 data in", 6: "item 0 computed", 7: "item 1 data in",
          8: "h ready (down)", 9: "down computed", 2: "resident units done", 10: "drained", 31: "exit",
          12: "mirror: epoch", 13: "mirror: all out"}
TICK_US = 0.01


def timeline(workload="c2", reps=10, warm=30, copies=8):
    import torch

    from .workload import DeviceLayer

    cfg = synth.CONFIGS[workload]
    layer = DeviceLayer(cfg, copies=copies, with_y32=False, diagnostics=False, stamps=True)
    layer.seal_empty_queue(1)
    waves = (layer.backend.max_workers + 1) * 4
    phases = {k: [] for k in PHASES}
    spans = {"down data in -> h ready": [], "h ready -> down computed": [], "down computed -> drained": [],
             "item 0 computed -> down data in": []}
    for rep in range(reps):
        for i in range(warm):
            layer.run_core(copy=i % copies, epoch=1)
        layer.stamps.zero_()
        layer.run_core(copy=rep % copies, epoch=1)
        torch.cuda.synchronize()
        st = layer.stamps.cpu().numpy().reshape(-1, 32)[:waves].astype(np.int64)
        t0 = st[:, 0][st[:, 0] > 0].min()
        for k in PHASES:
            v = st[:, k]
            phases[k].append((v[v > 0] - t0) * TICK_US)
        d = st[st[:, 9] > 0]
        data = np.where(d[:, 7] > 0, d[:, 7], d[:, 5])

        def span(name, later, earlier):
            ok = (later > 0) & (earlier > 0)   # walks that stamp both phases
            spans[name].append((later[ok] - earlier[ok]) * TICK_US)

        span("down data in -> h ready", d[:, 8], data)
        span("h ready -> down computed", d[:, 9], d[:, 8])
        span("down computed -> drained", d[:, 10], d[:, 9])
        two = d[:, 7] > 0
        span("item 0 computed -> down data in", d[two, 7], d[two, 6])
    status = layer.backend.status()
    layer.close()
    return cfg, waves, status, phases, spans, reps


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="c2")
    ap.add_argument("--reps", type=int, default=10)
    a = ap.parse_args()
    cfg, waves, status, phases, spans, reps = timeline(a.workload, a.reps)
    print(f"{cfg.name}: {waves} waves, status {status}; µs after the first wave's start")
    print("| phase | waves per launch | p10 | p50 | p90 | max |")
    print("|---|---|---|---|---|---|")
    for k in sorted(phases, key=lambda k: np.median(np.concatenate(phases[k])) if len(np.concatenate(phases[k])) else 0):
        v = np.concatenate(phases[k])
        if len(v):
            print(f"| {PHASES[k]} | {len(v) // reps} | {np.percentile(v, 10):.2f} | {np.percentile(v, 50):.2f} | "
                  f"{np.percentile(v, 90):.2f} | {v.max():.2f} |")
    print()
    print("| per-wave interval (waves with a down item) | p10 | p50 | p90 | max |")
    print("|---|---|---|---|---|")
    for k, parts in spans.items():
        v = np.concatenate(parts)
        if len(v):
            print(f"| {k} | {np.percentile(v, 10):.2f} | {np.percentile(v, 50):.2f} | {np.percentile(v, 90):.2f} | "
                  f"{v.max():.2f} |")


if __name__ == "__main__":
    main()
