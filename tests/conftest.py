import os
import sys
from pathlib import Path

import pytest

# The parity tests must exercise the native forward: a call it cannot take
# raises instead of running the native-torch fallback (tests of the fallback
# itself turn this off per model).
os.environ.setdefault("ENC_NATIVE_ONLY", "1")

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")
    config.addinivalue_line("markers", "slow: long-running (large shapes)")


def _gpu_available() -> bool:
    try:
        import torch
    except ImportError:
        return False
    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    import torch

    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before it touches the GPU, flushed, so a crash is attributable.
    if "gpu" in request.keywords:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
        sys.stdout.flush()
    yield
    if "gpu" in request.keywords and os.environ.get("ENC_TEST_SYNC", "1") == "1":
        import torch

        if torch.cuda.is_available():
            torch.cuda.synchronize()
