import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP extension")


@pytest.fixture
def gpu():
    """The GPU device; fails (does not skip) when the HIP extension is missing."""
    import torch

    import nibble_amd

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    if not nibble_amd.cuda_extension_available():
        raise RuntimeError(f"W4A16 HIP extension not loaded: {nibble_amd.cuda.extension_load_error()}")
    return torch.device("cuda:0")
