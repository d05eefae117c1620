import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    import torch

    return torch.device("cuda:0")


def pytest_runtest_logstart(nodeid, location):
    # Name the case before any GPU work so a crash that kills the process still identifies it.
    if os.environ.get("SPS_TRACE_TESTS"):
        print(f"\n[start] {nodeid}", flush=True)
