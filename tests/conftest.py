import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402  (torch first: the HIP libraries must use torch's HIP runtime)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import attention_amd

    # On a GPU box the HIP library must be the code under test, never skipped.
    assert attention_amd.is_cuda_extension_loaded(), "HIP op library failed to load"
    return torch.device("cuda:0")
