import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and the built libfarope.so")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Per-case errors of the GPU parity tests (max / mean absolute error and
    the bound each was held to), shown even under -q."""
    try:
        from tests import _report
    except ImportError:
        return
    if _report.LINES:
        terminalreporter.section("parity errors measured")
        for line in _report.LINES:
            terminalreporter.write_line(line)


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
