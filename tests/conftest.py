import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: tests that need an MI355X (HIP) device")
    config.addinivalue_line("markers", "phase9: theria's Phase 9 operator contract suite")
    config.addinivalue_line("markers", "boundary: known differentiation boundary tests")


@pytest.fixture(scope="session")
def hip_device():
    """The HIP device for gpu-marked tests; fails (not skips) when the kernels cannot run there."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    from theria_amd import _lib

    _lib.load()  # raises loudly if the kernel library is missing
    return torch.device("cuda:0")
