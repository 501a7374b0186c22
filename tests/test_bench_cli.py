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
