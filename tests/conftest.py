"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs everywhere (oracle vs golden vectors, host logic, C-ABI exports);
`-m gpu` needs a gfx950 GPU and calls the HIP library through its C ABI.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "rotor-rag_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


def _gpu_available():
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip():
    """The HIP backend on cuda:0.  GPU tests fail (not skip) when the library is
    missing on a machine that has a GPU."""
    if not _gpu_available():
        pytest.skip("no GPU visible")
    from rotor.gpu_ternary import HIPTernaryOps

    return HIPTernaryOps(0)
