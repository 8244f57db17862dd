import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; a GPU test fails loudly (never skips) when no device or no built library is present."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    from nanochat_amd import native

    native.hip_library()  # raises if the library is missing or stale
    return torch.device("cuda:0")
