"""Offline characterization of the CDNA4 kernel candidates and synthesis of the decision LUT.

LeanStream selects a kernel configuration per layer from an immutable table indexed by the
quantized remaining-I/O load at submission time (docs/kernel_selection.md): candidates are
measured offline on the target platform, the table is synthesized offline, and the runtime
only reads it (KernelSelector::select, O(1)). This module is that offline step for the
MI355X catalog (include/leanstream/hip_backend.h kHipCandidates).

Measurement of bucket q (of B): the layer's k active groups all go through the ready queue;
rem_q = floor((q + 1/2) k / B) of them are still unpublished when the layer is enqueued
(quantize_io_load(rem_q, k, B) == q), and a host publisher thread releases them after the
launch at a fixed gap (default 5 us, in the seeded ready order) -- the arrival of groups
that are still being staged. The figure of merit is the host wall time from the enqueue
call to the layer's completion word, the latency the decode loop sees. Each (bucket,
candidate) is run `trials` times over layer copies that together exceed the Infinity Cache;
the median decides, and ties within `tie_pct` percent keep the catalog default.

    python -m leanstream_amd.lut_sweep --workload c2 --out profiles/kernel_lut_sweep_c2.json
    python -m leanstream_amd.lut_sweep --header include/leanstream/hip_kernel_lut.h \\
        profiles/kernel_lut_sweep_c1.json profiles/kernel_lut_sweep_c2.json
"""
import argparse
import json
import math
import time
from pathlib import Path

import numpy as np

from . import synth
from .backend import MODE_PROGRESSIVE

BUCKETS = 8
MALL_BYTES = 256 * 2 ** 20
# kHipCandidates (include/leanstream/hip_backend.h): name, workers (0: all resident), entry
# point (0 fused, 1 split), group_batch, walk (unroll: 1 = the plain walk), down tile
# (tile_size: 256 = whole tiles)
CANDIDATES = ("hip_fused_w256", "hip_fused_resident", "hip_fused_w1024", "hip_split_w256", "hip_split_resident",
              "hip_fused_resident_pairs", "hip_fused_resident_plain", "hip_fused_resident_tiles")
CONFIGS = ((256, 0, 0, 0, 0), (0, 0, 0, 0, 0), (1024, 0, 0, 0, 0), (256, 1, 0, 0, 0), (0, 1, 0, 0, 0),
           (0, 0, 2, 0, 0), (0, 0, 0, 1, 0), (0, 0, 0, 0, 256))
DEFAULT_CANDIDATE = 5   # kHipDefault: the reference's ready-pair order
STAGED_MAX_WIDTH, QUARTERS_MAX_WIDTH, STAGED_GROUP = 4096, 2048, 64


def shape_walk(width, group_size):
    """The walk a batch-1 shape takes by default: staged (64-neuron groups, d <= 4096),
    packed (groups of at most 32 neurons) or plain."""
    if group_size == STAGED_GROUP and width <= STAGED_MAX_WIDTH:
        return "staged"
    return "packed" if group_size <= 32 else "plain"


def effective_configs(resident, width=4096, group_size=64):
    """(workers, entry, group_batch, walk, tile) each candidate launches with for a batch-1
    shape on this device -- worker counts clamped to the co-resident maximum, a walk or tile
    the shape does not offer replaced by what it launches instead -- and for each candidate
    the first candidate id with the same launch: identical launches are measured once. (The
    plain walk's own co-resident count may differ; it is always a launch of its own.)"""
    walk = shape_walk(width, group_size)
    eff = []
    for w, e, b, pw, tile in CONFIGS:
        plain = 1 if pw == 1 and walk != "plain" else 0
        tiles = 256 if tile == 256 and walk == "staged" and width <= QUARTERS_MAX_WIDTH and not plain else 0
        eff.append((min(w, resident) if w else resident, e, b, plain, tiles))
    first = [eff.index(x) for x in eff]
    return eff, first


def remaining_for_bucket(q, k, buckets=BUCKETS):
    """Unpublished groups at enqueue for bucket q: the midpoint of the bucket's range."""
    rem = int(math.floor((q + 0.5) * k / buckets))
    return max(0, min(k, rem))


def quantize_io_load(remaining, total, buckets=BUCKETS):
    """docs/kernel_selection.md: min(buckets - 1, floor(min(remaining, total) * buckets / total))."""
    if not total or not buckets:
        return 0
    return min(buckets - 1, (min(remaining, total) * buckets) // total)


def sweep(workload, trials=25, gap_ns=5000, copies=0, log=print):
    import torch

    from .workload import DeviceLayer

    cfg = synth.CONFIGS[workload]
    k = cfg.active
    active_bytes = cfg.algorithmic_bytes()
    copies = copies or max(2, math.ceil(1.5 * MALL_BYTES / active_bytes))
    # one backend; bucket c of this one-layer table selects candidate c
    table = [list(range(len(CANDIDATES)))]
    layer = DeviceLayer(cfg, copies=copies, with_y32=False, diagnostics=False, offline_table=table)
    stream = torch.cuda.current_stream().cuda_stream
    q = layer.queue
    order = synth.ready_order(k, cfg)
    rows = [synth.descriptors(cfg, layer.logical, source_kind=0) for _ in range(copies)]
    for c in range(copies):
        rows[c][:, 1] += c * cfg.groups
        rows[c][:, 2] += c * cfg.groups
    eff, first = effective_configs(layer.backend.max_workers, cfg.width, cfg.group_size)
    measured = sorted(set(first))
    rng = np.random.default_rng(0x5EED)
    epoch = 100
    times = np.zeros((BUCKETS, len(CANDIDATES), trials))
    step = 0
    for bucket in range(BUCKETS):
        rem = remaining_for_bucket(bucket, k)
        assert quantize_io_load(rem, k) == bucket
        before, after = order[:k - rem], order[k - rem:]
        offs = (np.arange(1, len(after) + 1, dtype=np.uint64) * np.uint64(gap_ns))
        for t in range(trials):
            for cand in rng.permutation(measured):   # a fresh order every trial
                cand = int(cand)
                epoch += 1
                copy = step % copies
                step += 1
                q.write_descriptors(rows[copy])
                q.reset(epoch)
                q.seal(k)
                for i in before:
                    q.publish(int(i))
                torch.cuda.synchronize()
                t0 = time.perf_counter_ns()
                layer.backend.enqueue(0, cand, epoch, layer.x, layer.y, stream, None, 0, q, MODE_PROGRESSIVE)
                pub = q.start_publisher(after, offs) if len(after) else None
                while not layer.backend.complete(0):
                    if time.perf_counter_ns() - t0 > 10 ** 10:   # the kernels' own waits end within 2 s
                        raise RuntimeError(f"candidate {cand} bucket {bucket}: no completion")
                t1 = time.perf_counter_ns()
                if pub:
                    pub.join()
                torch.cuda.synchronize()
                if layer.backend.status():
                    raise RuntimeError(f"candidate {cand} bucket {bucket}: status {layer.backend.status()}")
                times[bucket, cand, t] = (t1 - t0) / 1e3
        for c in range(len(CANDIDATES)):
            times[bucket, c] = times[bucket, first[c]]
        med = np.median(times[bucket], axis=1)
        log(f"{workload} bucket {bucket} (unpublished {rem}/{k}): " +
            ", ".join(f"{CANDIDATES[c]} {med[c]:.1f}" for c in range(len(CANDIDATES))))
    layer.close()
    return dict(workload=workload, name=cfg.name, width=cfg.width, group_size=cfg.group_size, active=k,
                buckets=BUCKETS, trials=trials, gap_ns=gap_ns, copies=copies, candidates=list(CANDIDATES),
                launches=[list(x) for x in eff], same_launch_as=first,
                remaining=[remaining_for_bucket(b, k) for b in range(BUCKETS)],
                median_us=np.median(times, axis=2).round(3).tolist(),
                p10_us=np.percentile(times, 10, axis=2).round(3).tolist(),
                p90_us=np.percentile(times, 90, axis=2).round(3).tolist())


def winners(result, tie_pct=2.0):
    """Per bucket: the fastest median; the default candidate when it is within tie_pct (or
    launches the same configuration)."""
    out = []
    first = result.get("same_launch_as", list(range(len(CANDIDATES))))
    for med in result["median_us"]:
        best = int(np.argmin(med))
        if first[best] == first[DEFAULT_CANDIDATE] or med[DEFAULT_CANDIDATE] <= med[best] * (1 + tie_pct / 100):
            best = DEFAULT_CANDIDATE
        out.append(best)
    return out


def write_header(path, results):
    lines = [
        "// Offline-measured CDNA4 kernel decision rows (generated by leanstream_amd/lut_sweep.py",
        "// from the sweeps in profiles/kernel_lut_sweep_*.json; do not edit by hand).",
        "// One row of io buckets per layer shape: entry q is the kHipCandidates id with the",
        "// lowest median enqueue-to-completion latency when quantize_io_load(remaining, k, 8) == q",
        "// at submission (docs/kernel_selection.md). A homogeneous model repeats the row for",
        "// every layer: hip_lut_rows(row, layers, out) fills a caller-owned [layers][8] table.",
        "#pragma once",
        "#include <stdint.h>",
        "#include \"leanstream/kernel_selector.h\"",
        "",
        "namespace leanstream::runtime::cdna4 {",
        "",
        f"inline constexpr uint32_t kLutBuckets = {BUCKETS};",
    ]
    for r in results:
        w = winners(r)
        lines.append(f"// {r['name']}: width {r['width']}, group {r['group_size']}, {r['active']} active groups; "
                     f"unpublished at enqueue per bucket {r['remaining']}")
        lines.append(f"inline constexpr uint8_t kLutD{r['width']}G{r['group_size']}[{BUCKETS}] = "
                     "{" + ", ".join(str(v) for v in w) + "};")
    lines += [
        "",
        "// Copies `row` into every one of `layers` rows of `out` ([layers][kLutBuckets]) and",
        "// returns the table view (borrowed: `out` must outlive the selector).",
        "inline KernelDecisionTable hip_lut_rows(const uint8_t* row, uint32_t layers, uint8_t* out) noexcept {",
        "    for (uint32_t l = 0; l < layers; ++l)",
        "        for (uint32_t q = 0; q < kLutBuckets; ++q) out[l * kLutBuckets + q] = row[q];",
        "    return {out, layers, kLutBuckets};",
        "}",
        "",
        "}  // namespace leanstream::runtime::cdna4",
        "",
    ]
    Path(path).write_text("\n".join(lines))


def write_markdown(path, results, commands):
    """The sweep summary of profiles/: per shape, the median latency of every candidate per
    bucket and the winner."""
    lines = ["# Kernel candidate sweep per io bucket (offline CDNA4 LUT)", "",
             "Command (one MI355X, each workload in its own process):", ""]
    lines += [f"    {c}" for c in commands]
    lines += ["", "Figure: median host wall time (µs) from the enqueue call to the layer's completion word, "
              f"{results[0]['trials']} trials in a fresh random candidate order each, over layer copies exceeding the "
              "Infinity Cache. Bucket q: all k groups go through the ready queue, rem_q = floor((q + 1/2) k / 8) of "
              "them unpublished at enqueue and then published 5 µs apart. Candidates whose launch is the same on "
              "MI355X for the shape are measured once (\"same as\"). Winner: fastest median, the default (5) when "
              "within 2%.", ""]
    for r in results:
        lines += [f"## {r['name']} (d = {r['width']}, groups of {r['group_size']}, k = {r['active']})", ""]
        same = [f"{CANDIDATES[c]} = {CANDIDATES[f]}" for c, f in enumerate(r["same_launch_as"]) if f != c]
        if same:
            lines += ["Same launch: " + "; ".join(same) + ".", ""]
        lines.append("| bucket | unpublished | " + " | ".join(CANDIDATES) + " | winner |")
        lines.append("|---" * (len(CANDIDATES) + 3) + "|")
        w = winners(r)
        for q, med in enumerate(r["median_us"]):
            lines.append(f"| {q} | {r['remaining'][q]} | " + " | ".join(f"{v:.1f}" for v in med) + f" | {w[q]} |")
        lines.append("")
        med = np.asarray(r["median_us"])
        gain = (med[:, DEFAULT_CANDIDATE] / med.min(axis=1) - 1) * 100
        arrival = np.asarray(r["remaining"]) * r["gap_ns"] / 1e3
        if all(x == DEFAULT_CANDIDATE for x in w):
            lines += [f"Every bucket keeps the default: no candidate beats it by more than {gain.max():.1f}% "
                      f"(the 2% tie margin). The latency follows the last publication "
                      f"({arrival[0]:.0f}-{arrival[-1]:.0f} µs after the enqueue across the buckets), which no "
                      "launch configuration can move.", ""]
        else:
            lines += [f"Buckets {[q for q, x in enumerate(w) if x != DEFAULT_CANDIDATE]} select another candidate "
                      f"(up to {gain.max():.1f}% below the default's median).", ""]
    Path(path).write_text("\n".join(lines))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="c2")
    ap.add_argument("--trials", type=int, default=25)
    ap.add_argument("--gap-ns", type=int, default=5000)
    ap.add_argument("--out")
    ap.add_argument("--header", help="write the C++ header from the sweep files given as arguments")
    ap.add_argument("--markdown", help="write the sweep summary from the sweep files given as arguments")
    ap.add_argument("sweeps", nargs="*")
    a = ap.parse_args()
    if a.header or a.markdown:
        results = [json.loads(Path(p).read_text()) for p in a.sweeps]
        if a.header:
            write_header(a.header, results)
        if a.markdown:
            cmds = [f"python -m leanstream_amd.lut_sweep --workload {r['workload']} --out {p}"
                    for r, p in zip(results, a.sweeps)]
            cmds.append("python -m leanstream_amd.lut_sweep --header include/leanstream/hip_kernel_lut.h "
                        "--markdown profiles/kernel_lut_sweep.md " + " ".join(a.sweeps))
            write_markdown(a.markdown, results, cmds)
        return
    r = sweep(a.workload, trials=a.trials, gap_ns=a.gap_ns, log=lambda m: print(m, flush=True))
    r["winners"] = winners(r)
    print(json.dumps({"workload": r["workload"], "winners": r["winners"]}), flush=True)
    if a.out:
        Path(a.out).write_text(json.dumps(r, indent=1) + "\n")


if __name__ == "__main__":
    main()
