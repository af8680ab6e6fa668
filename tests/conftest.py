import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "redline-tiny_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu on a machine that has one")


@pytest.fixture(scope="session")
def dev():
    """The GPU every gpu-marked test runs on; fails (does not skip) when there is none."""
    import torch
    assert torch.cuda.is_available(), "gpu-marked tests need a ROCm GPU"
    from rlbfp import _lib
    _lib.check(_lib.lib().rl_device_check())
    return torch.device("cuda:0")
