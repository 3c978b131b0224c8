import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libvx_attn.so")
    config.addinivalue_line("markers", "slow: full-size configurations")


def pytest_collection_modifyitems(config, items):
    # GPU tests print the case they run so a box that dies mid-run still names it.
    pass


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from vidax_amd import _lib
    _lib.lib()  # raises if the library was not built
    return torch.device("cuda:0")
