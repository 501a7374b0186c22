"""bench.py's command-line contract on the CPU: one GPU only (--gpus above 1 exits with a
message and status 2 before touching the GPU), and every workload the default run times
beside the headline names a configuration the package defines."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_secondary_workloads_name_known_configs():
    sys.path.insert(0, str(ROOT))
    import bench
    from leanstream_amd import synth

    keys = [k for k, _, _ in bench.SECONDARY]
    assert len(keys) == len(set(keys)) and "c2" not in keys   # the headline is not repeated
    for key, steps, warmup in bench.SECONDARY:
        assert key in synth.CONFIGS or key in synth.STREAMS, key
        assert steps > 0 and warmup >= 0


def test_a_failing_secondary_workload_does_not_lose_the_others(monkeypatch):
    sys.path.insert(0, str(ROOT))
    import bench

    def fake_layer(cfg, steps, warmup, **kw):
        if "llama70b" in cfg.name:
            raise AssertionError("device status 1")
        return {"us": 10.0}

    def fake_decode(sc, steps, warmup, **kw):
        raise RuntimeError("ETIMEDOUT")

    monkeypatch.setattr(bench, "timed_layer", fake_layer)
    monkeypatch.setattr(bench, "decode_steps", fake_decode)
    out = bench.secondary_workloads()
    assert set(out) == {k for k, _, _ in bench.SECONDARY}
    assert "error" in out["c4"] and "error" in out["c4b4"] and "error" in out["c3"]
    assert out["c1"]["us_per_layer"] == 10.0 and out["c5"]["us_per_layer"] == 10.0


def test_a_failing_chain_does_not_lose_the_other(monkeypatch):
    """The default run's pipelined figures: one per shape, each failure reported in its own
    entry while the other stands."""
    sys.path.insert(0, str(ROOT))
    import bench

    def fake_chain(cfg, steps, warmup, layers=36, **kw):
        if cfg.width == 1024:
            raise AssertionError("device status 1")
        return {"us": 12.0}

    monkeypatch.setattr(bench, "timed_chain", fake_chain)
    monkeypatch.setattr(bench, "timed_dependent", lambda cfg, steps, warmup, layers=36: {"us": 20.0})
    out = bench.pipelined_workloads()
    assert set(out) == {"c2", "c1"}
    assert out["c2"]["us_per_layer"] == 12.0 and out["c2"]["layers_per_launch"] == 36
    assert out["c2"]["per_launch_dependent_us_per_layer"] == 20.0
    assert "error" in out["c1"]


def test_control_plane_timing_runs_on_the_host():
    """The C1 layer's control plane (Runtime / WeightManager / ExecutionQueue, no GPU) times on
    one host thread and reports every active group published."""
    sys.path.insert(0, str(ROOT))
    import bench

    r = bench.control_plane_timing(seconds=0.2)
    assert r["groups"] == 64 and r["active"] == 16 and r["threads"] == 1
    assert r["layers"] > 0 and 0 < r["us_per_layer"] < 1000
