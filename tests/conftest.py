import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "mojo-adreno_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


_GPU = None


def gpu_available() -> bool:
    global _GPU
    if _GPU is None:
        import torch
        _GPU = bool(torch.cuda.is_available())
    return _GPU


@pytest.fixture
def dev():
    if not gpu_available():
        pytest.skip("no GPU visible")
    import torch
    import aq  # noqa: F401  (registers torch.ops.aq.*)
    return torch.device("cuda:0")


def pytest_runtest_setup(item):
    # Name the case on stdout before any GPU work, so a run that dies mid-test still says which one it was.
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {item.nodeid}", flush=True)
        os.environ.setdefault("AQ_TEST_CASE", item.nodeid)
