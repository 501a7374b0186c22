"""The claim-log checker (tests/claims.py) on logs of the reference claim loop and on
planted mistakes (CPU only)."""
import numpy as np
import pytest

from claims import STATIC, check_claim_log, simulate_claims, static_log


@pytest.mark.parametrize("total,workers", [(1, 4), (2, 4), (16, 4), (37, 8), (58, 511), (90, 3)])
def test_reference_claim_loop_logs_pass(total, workers):
    rng = np.random.default_rng(total * 31 + workers)
    for trial in range(20):
        steps = np.sort(rng.integers(1, total + 1, size=rng.integers(1, 6)))
        steps = np.append(steps, total)
        log = simulate_claims(total, 2, workers, list(steps), rng)
        assert check_claim_log(log, total, 2, workers) == "claimed"


@pytest.mark.parametrize("total,workers", [(1, 4), (16, 4), (37, 8), (58, 511), (90, 3)])
def test_static_pairs_pass(total, workers):
    log = static_log(total, 2, workers)
    assert check_claim_log(log, total, 2, workers) == "static"
    # taken in any order (timing), still valid
    e = log.reshape(-1, 4)[::-1].reshape(-1)
    assert check_claim_log(e, total, 2, workers) == "static"


def _mutate(log, fn):
    e = log.reshape(-1, 4).astype(np.int64).copy()
    fn(e)
    return e.astype(np.uint64).reshape(-1)


def test_single_claimer_log_passes():
    """Claimed ranges taken by one claimer (worker index W, the queue mirror) as positions
    become ready: the reference's ranges, in publication order."""
    e = []
    head = 0
    for ready in (3, 4, 9, 16):
        while head < ready:
            end = min(head + 2, ready)
            e.append((head, end - head, ready, 4))
            head = end
    assert check_claim_log(np.asarray(e, dtype=np.uint64).reshape(-1), 16, 2, 4) == "claimed"


def test_planted_mistakes_fail():
    rng = np.random.default_rng(7)
    log = simulate_claims(16, 2, 4, [3, 9, 16], rng)
    bad = {
        "overlap": lambda e: e.__setitem__((1, 0), e[1, 0] - 1),
        "gap": lambda e: e.__setitem__((-1, 1), e[-1, 1] - 1) if e[-1, 1] > 1 else e.__setitem__((-1, 0), e[-1, 0] + 1),
        "triple": lambda e: e.__setitem__((0, 1), 3),
        "short claim": lambda e: e.__setitem__((0, 2), 16) if e[0, 1] == 1 else e.__setitem__((0, 1), 1),
        "not ready": lambda e: e.__setitem__((0, 2), e[0, 0]),
        "worker": lambda e: e.__setitem__((0, 3), 5),   # 4 = the single claimer (the mirror) is allowed
    }
    for name, fn in bad.items():
        with pytest.raises(AssertionError):
            check_claim_log(_mutate(log, fn), 16, 2, 4)
            raise RuntimeError(f"{name} not detected")
    st = static_log(16, 2, 4)
    for name, fn in {"owner": lambda e: e.__setitem__((0, 3), (e[0, 3] + 1) % 4),
                     "mirror owns a static range": lambda e: e.__setitem__((0, 3), 4),
                     "odd start": lambda e: (e.__setitem__((0, 0), 1), e.__setitem__((0, 1), 1)),
                     "mixed paths": lambda e: e.__setitem__((0, 2), 16)}.items():
        with pytest.raises(AssertionError):
            check_claim_log(_mutate(st, fn), 16, 2, 4)
            raise RuntimeError(f"{name} not detected")
    with pytest.raises(AssertionError):       # a position missing
        check_claim_log(static_log(16, 2, 4)[:-4], 16, 2, 4)
    assert STATIC == 0xFFFFFFFF
