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


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Worst err / bar ratio per GPU test family (tests/bars.py); also written as JSON to $THERIA_MARGIN_LOG."""
    import json
    import os

    try:
        from bars import MARGINS
    except ImportError:
        return
    if not MARGINS:
        return
    terminalreporter.write_sep("-", "worst err / bar per test family")
    for fam, (ratio, what) in sorted(MARGINS.items(), key=lambda kv: -kv[1][0]):
        terminalreporter.write_line(f"{ratio:7.3f}  {fam}: {what}")
    path = os.environ.get("THERIA_MARGIN_LOG")
    if path:
        with open(path, "w") as f:
            json.dump({k: {"ratio": v[0], "where": v[1]} for k, v in MARGINS.items()}, f, indent=1, sort_keys=True)
