import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library (run with -m gpu)")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; GPU tests fail loudly if the HIP library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from kiv_amd import _native

    _native.lib()  # raises when libkiv_hip.so has not been built
    return torch.device("cuda", 0)
