from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and the built HIP library")


@pytest.fixture(scope="session")
def gpu_device():
    """The GPU tests must run on a GPU: fail (not skip) when none is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a ROCm GPU")
    from flare_amd import _native

    _native.library()  # raises if the HIP library was not built
    return torch.device("cuda", 0)


@pytest.fixture()
def no_device_errors(gpu_device):
    """Assert that the kernels of a test recorded no out-of-range / guard errors."""
    import torch

    from flare_amd import _native

    def check(expected: int = 0):
        torch.cuda.synchronize()
        bits = _native.library().flare_take_device_errors(None)
        assert bits == expected, f"device error bits {bits} (expected {expected})"

    check_clear = _native.library().flare_take_device_errors(None)  # clear leftovers
    del check_clear
    return check
