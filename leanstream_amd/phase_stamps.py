"""Per-wave phase timeline of one persistent layer launch, from the kernels' own stamps.

With a stamps buffer bound (HipLayerBuffers::stamps), every wave of the fused kernel writes
the device's 100 MHz clock (s_memrealtime) at fixed points of its walk (lsamd::StampPhase in
leanstream_amd/csrc/mlp_args.h). This diagnostic runs a workload's layer back to back over
rotated copies, then stamps one launch after each batch of warm launches, and prints each
phase's time after the first wave's start (percentiles over waves and repetitions), plus
per-wave intervals of the waves that hold a down item.

    python -m leanstream_amd.phase_stamps --workload c2
    python -m leanstream_amd.phase_stamps --workload chain --reps 3
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


# Chain stamps (per layer and wave, lsamd::ChainStamp and StampPhase in mlp_args.h).
CHAIN_PHASES = ((14, "first item issued"), (16, "input in LDS (stager)"), (6, "first gate/up item computed"),
                (5, "first down item data in"), (9, "first down item computed"), (10, "last item drained"))
CHAIN_DONE = 18   # the supervisor's stamp: every wave out of the layer, completion word stored


def chain_timeline(workload="chain", layers=36, reps=3):
    """Phase stamps of chain launches (ls_hip_set_chain_stamps): per layer l, each phase in µs
    after layer l - 1's last column was written (the last wave's drain of that layer: every
    input word of layer l exists from then on), percentiles over the waves that reach it,
    then the median over layers 1 .. layers - 2 and repetitions. A negative "first item
    issued" is a layer whose weights were requested before the layer before it had
    finished; "layer complete" is the supervisor's count-out, which trails the data (waves
    count out of a layer lazily, after their next item's data wait)."""
    import torch

    from .workload import DeviceLayer

    cfg = synth.CONFIGS["c2" if workload == "chain" else "c1"]
    rows = {name: [] for _, name in CHAIN_PHASES}
    rows["layer complete"] = []
    issued_before = []
    layer = DeviceLayer(cfg, copies=layers, with_y32=False, diagnostics=False)
    outputs = layer.chain_outputs(layers)
    norm = layer.chain_norm_weights(layers)
    blocks = layer.backend.chain_blocks(layer.chain_layers(list(range(layers)), outputs, output32=False, norm=norm))
    sid = torch.cuda.current_stream().cuda_stream
    nw = (layer.backend.chain_workers + 1) * 4
    stamps = torch.zeros(layers * nw * 32, dtype=torch.int64, device="cuda")
    snaps = []
    for _ in range(reps):
        for _ in range(3):   # warm launches, then one stamped launch
            layer.backend.enqueue_chain(blocks, sid)
        layer.backend.set_chain_stamps(stamps, layers)
        stamps.zero_()
        layer.backend.enqueue_chain(blocks, sid)
        torch.cuda.synchronize()
        layer.backend.set_chain_stamps(None, 0)
        snaps.append(stamps.cpu().numpy().reshape(layers, nw, 32).astype(np.int64))
    status = layer.backend.status()
    layer.close()
    assert status == 0, f"device status {status}"
    for st in snaps:
        done = st[:, nw - 4, CHAIN_DONE]   # wave 0 of the supervisor workgroup
        for i in range(1, layers - 1):
            t0 = st[i - 1, :, 10].max()
            for k, name in CHAIN_PHASES:
                v = st[i, :, k]
                v = (v[v > 0] - t0) * TICK_US
                if len(v):
                    rows[name].append([np.percentile(v, 10), np.percentile(v, 50), np.percentile(v, 90), v.max()])
            rows["layer complete"].append([(done[i] - t0) * TICK_US] * 4)
            iss = st[i, :, 14]
            iss = iss[iss > 0]
            issued_before.append(float(np.mean(iss < t0)))
    return cfg, rows, float(np.median(issued_before))


def chain_main(a):
    cfg, rows, before = chain_timeline(a.workload, a.layers, a.reps)
    print(f"chain of {a.layers} {cfg.name} layers; µs after the previous layer's last column (median over layers)")
    print("| phase | p10 | p50 | p90 | max |")
    print("|---|---|---|---|---|")
    for name, v in rows.items():
        if v:
            m = np.median(np.array(v), axis=0)
            print(f"| {name} | {m[0]:.2f} | {m[1]:.2f} | {m[2]:.2f} | {m[3]:.2f} |")
    print()
    print(f"waves whose first item of a layer was issued before the previous layer's last column: {before * 100:.1f}%")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="c2", help="a layer configuration, or chain / c1chain")
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--layers", type=int, default=36, help="chain workloads: layers per launch")
    ap.add_argument("--copies", type=int, default=8, help="layer copies the warm launches rotate over")
    a = ap.parse_args()
    if a.workload in ("chain", "c1chain"):
        chain_main(a)
        return
    cfg, waves, status, phases, spans, reps = timeline(a.workload, a.reps, copies=a.copies)
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
