import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Measured parity errors of the checks that report them (tests/_tol.py)."""
    from tests._tol import MARGINS
    if not MARGINS:
        return
    terminalreporter.write_sep("-", "parity margins: max|y - y_ref| / max|y_ref| (or element-wise)")
    for name, err, tol in MARGINS:
        terminalreporter.write_line(f"{name:<60s} {err:9.2e}  (tolerance {tol:.0e}, {err / tol:5.1%})")
