import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the device)")


def pytest_collection_modifyitems(config, items):
    # A GPU run must only launch prebuilt code objects: a cache miss is an
    # error, never a silent hipcc run on the box.
    if any(item.get_closest_marker("gpu") for item in items):
        os.environ.setdefault("TCA_JIT", "0")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from tcacomp_amd import _lib
    _lib.check(_lib.lib().tca_rt_init(0))
    return torch.device("cuda:0")
