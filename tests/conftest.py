import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu_lib():
    """The C-ABI library on a GPU, or a skip when there is no GPU. On a machine with a GPU a
    missing or unloadable library is an error, never a skip."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vllm_sly_radiance_amd import _native
    return _native.lib()
