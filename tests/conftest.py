"""Test configuration: import paths of the package and the oracle, and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle checks, the host logic and the C-ABI load checks on the CPU; ``-m gpu`` runs the
parity tests of the gfx950 kernels against the oracle (they need a ROCm GPU and the built library).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "eagle-4_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (gfx950) and the built libeagle4_amd.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda")


def announce(name: str) -> None:
    """Names the case about to run on the GPU (flushed, so a failing run's log says which one)."""
    print(f"[gpu case] {name}", flush=True)
