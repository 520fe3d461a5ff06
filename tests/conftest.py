import os
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(42)
    np.random.seed(42)
    yield


def pytest_collection_modifyitems(config, items):
    # GPU tests need a device; fail loudly (not skip) if -m gpu was requested
    # on a host without one, skip otherwise.
    if torch.cuda.is_available():
        return
    marker_expr = config.getoption("-m") or ""
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords and "not gpu" not in marker_expr and marker_expr != "gpu":
            item.add_marker(skip)
