import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 for GPU tests; fails loudly (no CPU fallback) when the GPU or library is absent."""
    import torch
    from helixml_amd import _ffi
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    _ffi.lib()  # raises if libhelix_hip.so is not built
    _ffi.call("hx_init", 0)
    return torch.device("cuda:0")
