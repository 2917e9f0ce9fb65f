import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


@pytest.fixture(scope="session")
def gpu_lib():
    """The HIP library, loaded once; GPU tests fail loudly if it is missing."""
    import torch  # noqa: F401  (initializes the ROCm runtime the same way the benchmark does)
    from heliox_amd import lib
    return lib()
