import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a real MI355X (gfx950) and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch import failure
        return False


@pytest.fixture(scope="session")
def hip_lib():
    """The built HIP library, loaded through the C-ABI loader (GPU tests)."""
    if not gpu_available():
        pytest.skip("no GPU visible")
    from rwkv7m_amd.kernels import wkv_hip
    return wkv_hip.load_library()
