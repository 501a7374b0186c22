"""Claim-log checks for queue consumers that take positions in ranges (the ready pairs of
LeanStream backends/triton/persistent.py:59-90).

A log entry is (first, count, ready, worker) -- one per range a worker took, in the
order taken (the layout of include/leanstream/hip_backend.h HipLayerBuffers::claim_log).

All-ready launches (ready == STATIC): worker w takes the descriptor-index ranges
[batch (w + k W), +batch) for k = 0, 1, ... (persistent.py:63-69, batch 2).
Progressive launches: a worker claims [head, min(head + batch, ready)) of the publication
positions by compare-and-swap on the claim head (persistent.py:71-87), so the heads rise
in claim order and the ranges are contiguous; which worker wins is timing-dependent (a
consumer may also take them with one claimer -- logged as worker index `workers`, the
queue mirror of the MI355X kernels -- and deal their items to every worker).
"""
import numpy as np

STATIC = 0xFFFFFFFF


def entries(log_words):
    """Log entries with a nonzero count (the buffer is zeroed before a launch)."""
    e = np.asarray(log_words, dtype=np.uint64).reshape(-1, 4)
    return e[e[:, 1] > 0]


def check_claim_log(log_words, total, batch, workers):
    """Raise AssertionError unless the log is a valid range consumption of `total` queue
    positions in ranges of `batch` by `workers` workers. Returns 'static' or 'claimed'."""
    e = entries(log_words)
    assert total == 0 or len(e), "no entries"
    if total == 0:
        assert len(e) == 0
        return "empty"
    kinds = set(int(r) == STATIC for r in e[:, 2])
    assert len(kinds) == 1, "a launch takes one path"
    static = kinds.pop()
    order = np.argsort(e[:, 0], kind="stable")
    e = e[order]
    first, count, ready, worker = (e[:, i].astype(np.int64) for i in range(4))
    assert np.all(worker < (workers if static else workers + 1)), "worker index out of range"
    # every position exactly once, union [0, total)
    covered = np.zeros(total, dtype=np.int64)
    for f, c in zip(first, count):
        assert 0 <= f and f + c <= total, ("range outside the queue", f, c)
        covered[f:f + c] += 1
    assert np.all(covered == 1), "a position taken twice or never"
    # contiguous ranges in head order
    assert first[0] == 0
    assert np.all(first[1:] == first[:-1] + count[:-1]), "ranges are not contiguous"
    if static:
        assert np.all(first % batch == 0), "static ranges start at multiples of the batch"
        assert np.all(count == np.minimum(batch, total - first)), "static range length"
        assert np.all(worker == (first // batch) % workers), "static ranges belong to worker (first / batch) % W"
        return "static"
    assert np.all(ready > first), "claimed a position not yet ready"
    assert np.all(ready <= total)
    assert np.all(count == np.minimum(batch, ready - first)), "claim is [head, min(head + batch, ready))"
    return "claimed"


def simulate_claims(total, batch, workers, ready_steps, rng):
    """The reference's claim loop (persistent.py:71-87) with a random interleaving of
    workers: ready_steps are the ready counts published over time (non-decreasing, last ==
    total). Returns the log (flat words)."""
    head, log, step = 0, [], 0
    ready = ready_steps[0]
    active = list(range(workers))
    while active:
        w = active[rng.integers(len(active))]
        if rng.random() < 0.3 and step + 1 < len(ready_steps):
            step += 1
            ready = ready_steps[step]
        if head >= total:
            active.remove(w)
        elif head < ready:
            end = min(head + batch, ready)
            log.append((head, end - head, ready, w))
            head = end
    return np.asarray(log, dtype=np.uint64).reshape(-1)


def static_log(total, batch, workers):
    """The all-ready ranges of every worker (persistent.py:63-69)."""
    log = []
    for w in range(workers):
        for first in range(batch * w, total, batch * workers):
            log.append((first, min(batch, total - first), STATIC, w))
    return np.asarray(log, dtype=np.uint64).reshape(-1)
