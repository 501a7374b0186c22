"""I/O admission parity with LeanStream's O_DIRECT engine (CPU).

tests/golden/staging_trace.cpp drives a WeightManager through its transport with every
read or copy held, released or failed by a script, and prints group states, staging
slots, read requests, queue words, publication order, descriptors, return codes and a
checksum of every staged slot. tests/golden/staging_trace.txt is what LeanStream's own
WeightManager prints on its built-in engine (src/io/stream_io.cpp with its
STREAM_TESTING read hook; tests/golden/make_staging_trace.sh). HostStagingIO must
reproduce it line for line: rank replacement, non-preemptive admission under the queue
depth, the terminal error word, recovery in a new epoch and the slot placement.
"""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden" / "staging_trace.txt"
DRIVER = ROOT / "tests" / "golden" / "staging_trace.cpp"
SOURCES = [ROOT / "leanstream_amd" / "csrc" / "runtime" / f
           for f in ("execution_queue.cpp", "weight_manager.cpp", "host_staging_io.cpp")]


def _run(tmp_path, name, extra=()):
    exe = tmp_path / name
    cmd = ["g++", "-O1", "-std=c++17", "-UNDEBUG", f"-I{ROOT / 'include'}", *extra, str(DRIVER),
           *map(str, SOURCES), "-lpthread", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120)


def test_host_staging_reproduces_reference_admission_trace(tmp_path):
    out = _run(tmp_path, "staging_mine").stdout.splitlines()
    want = GOLDEN.read_text().splitlines()
    for i, (a, b) in enumerate(zip(out, want)):
        assert a == b, f"first difference at line {i + 1}: got {a!r}, reference {b!r}"
    assert len(out) == len(want) and want[-1] == "== end"


def test_host_staging_trace_is_race_free(tmp_path):
    """The same scenarios under ThreadSanitizer: no report, same trace."""
    probe = subprocess.run(["g++", "-fsanitize=thread", "-x", "c++", "-", "-o", str(tmp_path / "probe")],
                           input="int main(){return 0;}", text=True, capture_output=True)
    if probe.returncode != 0:
        pytest.skip("ThreadSanitizer runtime not available")
    res = _run(tmp_path, "staging_tsan", ("-g", "-fsanitize=thread"))
    assert "ThreadSanitizer" not in res.stderr, res.stderr[:4000]
    assert res.stdout.splitlines() == GOLDEN.read_text().splitlines()


def test_staging_golden_is_current_with_the_reference_build():
    """Where LeanStream's sources are present (not on GPU test machines), the committed fixture
    must still be what the reference engine prints."""
    if not Path(os.environ.get("LEANSTREAM_REFERENCE", "/root/reference")).is_dir():
        pytest.skip("reference sources not present")
    ref = ROOT / "oracle" / "_ref" / "staging_trace_ref"
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "ref-staging"], check=True, capture_output=True)
    out = subprocess.run([str(ref)], check=True, capture_output=True, text=True, timeout=120).stdout.splitlines()
    assert out == GOLDEN.read_text().splitlines()
