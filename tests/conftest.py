"""Shared fixtures.  Tests marked ``gpu`` need a gfx950 device; everything
else runs on the CPU (oracle pinning, host logic, ABI load/export checks)."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "drama3-studio_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    return torch.device("cuda", 0)


def print_case(*parts):
    """Name the case before a GPU step so a fault can be attributed."""
    print("[case]", *parts, flush=True)
    os.environ["DMOE_LAST_CASE"] = " ".join(str(p) for p in parts)
