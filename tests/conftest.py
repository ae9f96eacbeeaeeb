import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "gemma4-moe-flash-mlx-turbo_amd"
for p in (ROOT, PKG, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libfmkv.so")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip on machines without a HIP device; fail loudly if the library is missing."""
    if not gpu_available():
        pytest.skip("no HIP device")
    import fmkv

    fmkv.load_library()  # raises when libfmkv.so was not built
    return fmkv


@pytest.fixture(scope="session")
def ora():
    import oracle

    oracle.lib()
    return oracle
