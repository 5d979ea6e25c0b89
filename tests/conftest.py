import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "oracle"), os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def torch_mod():
    import torch

    return torch


@pytest.fixture(scope="session")
def dev():
    """The GPU as a torch device. A gpu-marked test on a machine without one fails."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test on a machine without a HIP device")
    from relay_amd import _lib

    _lib.require_device()
    return torch.device("cuda:0")
