import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "my-inference-engine_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmi_fa2.so)")


def gpu_available():
    import torch
    return torch.cuda.is_available()


@pytest.fixture(autouse=True)
def _skip_gpu_without_device(request):
    if request.node.get_closest_marker("gpu") and not gpu_available():
        pytest.skip("no GPU in this environment")


def announce(msg):
    """Print-and-flush a line naming the case before a GPU step (shows with pytest -s)."""
    sys.__stdout__.write(msg + "\n")
    sys.__stdout__.flush()
