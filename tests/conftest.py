import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: larger CPU oracle cases")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Parity margins of every GPU-vs-oracle comparison, per tensor."""
    try:
        from tests.helpers import MARGINS, margin_summary
    except Exception:
        return
    if MARGINS:
        terminalreporter.write_sep("-", "parity margins (err / bound, 1.0 = at the tolerance)")
        terminalreporter.write_line(margin_summary())
