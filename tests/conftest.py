import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built liblaguna_hip.so")
    config.addinivalue_line("markers", "slow: full-size case (seconds of oracle work)")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _name_the_case(request):
    # Print the case name before it runs so a GPU failure is attributable from the log tail.
    if "gpu" in request.node.keywords:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
