"""pytest setup: the `gpu` marker and import paths.

`-m "not gpu"` runs on any machine (oracle pinning, host logic, ABI symbols);
`-m gpu` needs an MI355X and the built libmhc_amd.so.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "minimind-mhc_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libmhc_amd.so")


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible ROCm device")
    return torch.device("cuda:0")
