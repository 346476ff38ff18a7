import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


def rel_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    """Frobenius-norm relative error ||x - ref|| / ||ref|| in float64."""
    x = x.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    den = ref.norm().item()
    num = (x - ref).norm().item()
    return num / den if den > 0 else num


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from yanchor_amd import _native
    _native.lib()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")
