import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "qwen-mlx_amd"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and lib/libgdn.so")


@pytest.fixture(scope="session")
def gpu():
    """Skips nothing: a gpu-marked test on a machine without the GPU or the
    built library fails loudly."""
    import torch

    assert torch.cuda.is_available(), "gpu test run without a visible GPU"
    import gdn_amd

    gdn_amd.load()
    return torch.device("cuda:0")
