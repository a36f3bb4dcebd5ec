import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library and a visible GPU. GPU tests fail loudly without the library:
    nothing falls back to the CPU."""
    import torch

    from raceline_amd import lib

    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to a test marked gpu")
    lib.load()  # raises if libraceline_amd.so is missing
    return torch.device("cuda:0")
