import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
if str(ROOT / "tests") not in sys.path:
    sys.path.insert(0, str(ROOT / "tests"))

PKG = "collaborative-edge-system_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU")


def pytest_collection_modifyitems(config, items):
    # GPU tests are skipped only where no GPU exists at all; on a GPU machine a missing
    # kernel library makes them fail.
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def cea():
    return importlib.import_module(PKG)


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
