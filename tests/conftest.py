import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libpufferhip.so)")


@pytest.fixture(scope="session")
def gpu():
    """Skips without a visible GPU; on a GPU box, fails loudly if the HIP library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from pufferlean_amd import _lib
    _lib.lib()  # raises if libpufferhip.so was not built
    return torch.device("cuda:0")
