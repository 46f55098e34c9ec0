"""Shared test setup: the `gpu` marker, repo on sys.path, device fixture."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def gpu(dev):
    from crucible_amd.gpu import Gpu

    return Gpu(0)


@pytest.fixture
def tune():
    """set_tuning for one test: every key the test sets returns to its previous value."""
    from crucible_amd import _lib
    from crucible_amd.gpu import set_tuning

    lib = _lib.load()
    saved = {name: lib.crucible_attn_get_tuning(key) for name, key in _lib.TUNE_KEYS.items()}
    yield set_tuning
    for name, key in _lib.TUNE_KEYS.items():
        _lib.check(lib.crucible_attn_set_tuning(key, saved[name]))
