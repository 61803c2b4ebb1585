import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libbrx.so")


@pytest.fixture(scope="session")
def gpu():
    """Initialise libbrx on cuda:0; the GPU tests fail loudly if it cannot."""
    import torch

    from bigrig_amd import lib
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    lib.init(0)
    return torch.device("cuda:0")
