import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """The opened device (tessel_amd's C ABI); fails loudly without the library."""
    import tessel_amd

    tessel_amd.open()
    return tessel_amd
