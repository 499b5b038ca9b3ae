"""Shared fixtures. GPU tests carry @pytest.mark.gpu; everything else runs on CPU."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


@pytest.fixture(scope="session")
def flint():
    """The loaded libflint.so; fails loudly when it has not been built."""
    from flint_amd.flint_lib import Flint

    return Flint()


@pytest.fixture(scope="session")
def cuda():
    """Asserts a HIP device is present (GPU tests only): no CPU fallback exists."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a HIP device"
    return torch.device("cuda:0")


@pytest.fixture
def tune(flint):
    """tune(name, value) sets one plan override (flint_set_tuning) for this
    test; value None clears it. Every override the test set is cleared after
    it, so later tests run the default plans."""
    names = set()

    def set_(name, value):
        flint.set_tuning(name, value)
        names.add(name)

    yield set_
    for name in names:
        flint.set_tuning(name, None)
