import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run on the GPU box")


@pytest.fixture(scope="session")
def oracle():
    from q4k_ref import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def q4k():
    import mtlqwen_amd
    return mtlqwen_amd


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; a GPU test fails (not skips) when it is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device (run with -m 'not gpu' on CPU hosts)"
    import mtlqwen_amd  # noqa: F401  (fails loudly if libq4k.so is missing)
    return torch.device("cuda:0")
