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


def assert_states_close(got, want, rel: float = 1e-4) -> None:
    """fp32 recurrent states within ``rel`` relative error, entry by entry:
    ``|got - want| <= rel * (|want| + 1e-3 * max|want|)``. The floor at a thousandth of the largest entry covers
    entries that are residues of cancellation: their error is the rounding of the larger terms that cancelled, so it
    scales with the state, not with the entry. With ``rel`` 1e-4 the absolute floor is 1e-7 * max|want|."""
    import torch

    g, w = got.detach().cpu().double(), want.detach().cpu().double()
    assert g.shape == w.shape, (g.shape, w.shape)
    scale = w.abs().max().item() if w.numel() else 0.0
    err = (g - w).abs()
    bound = rel * (w.abs() + 1e-3 * scale)
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(f"{int(bad.sum())} of {w.numel()} state entries beyond {rel} relative: worst at flat "
                             f"index {i}, got {g.flatten()[i].item():.9g}, want {w.flatten()[i].item():.9g} "
                             f"(state scale {scale:.3g})")
