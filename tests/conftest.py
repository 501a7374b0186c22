import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    # Load what is built; build only what is missing.
    if not (ROOT / "oracle" / "liboracle.so").is_file():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    if not (ROOT / "leanstream_amd" / "libleanstream_hip.so").is_file():
        subprocess.run(["make", "-s", "-j8", "-C", str(ROOT / "leanstream_amd" / "csrc")], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch
