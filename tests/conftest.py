import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests need the built library (no fallback) and a gfx950 device."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    from bongard_amd import _lib

    _lib.lib()  # raises if the library is not built
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert name.startswith("gfx950"), f"expected gfx950, got {name}"
    return torch.device("cuda:0")
