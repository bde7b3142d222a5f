import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu_available():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible to torch")
    return True


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Print the achieved parity errors of every check that ran."""
    from tests._tolerance import summary_lines

    lines = summary_lines()
    if lines:
        terminalreporter.section("parity errors")
        for ln in lines:
            terminalreporter.write_line(ln)
