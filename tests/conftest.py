"""pytest configuration: the ``gpu`` marker, the ``slow`` gate and import paths.

GPU tests carry ``@pytest.mark.gpu``; the CPU suite runs with ``-m "not gpu"``.
Large cases are marked ``slow`` and skipped unless ``--runslow`` is given (the
reference suite gates its 8K prefill cases the same way, conftest.py:11-32 of
the reference).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_addoption(parser):
    parser.addoption("--runslow", action="store_true", default=False,
                     help="run slow (large) cases")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: large case; skipped unless --runslow is given")


def pytest_collection_modifyitems(config, items):
    if config.getoption("--runslow"):
        return
    skip_slow = pytest.mark.skip(reason="slow case; pass --runslow to run")
    for item in items:
        if "slow" in item.keywords:
            item.add_marker(skip_slow)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """One line per parity check of the session: the figures against the oracle
    (max_abs, mean_abs, check_result) and against the exact value (the
    reference's check_result share of the device and of the oracle, and the
    mean / max errors of both)."""
    try:
        from tests.gpu_helpers import FIGURES
    except Exception:  # noqa: BLE001 -- torch-less environments
        return
    if not FIGURES:
        return
    tr = terminalreporter
    tr.section("parity figures (device vs oracle | check_result vs exact: device / oracle / needed)")
    for f in FIGURES:
        line = (f"{f['case']}: max_abs={f['max_abs']:.2e} mean_abs={f['mean_abs']:.2e} "
                f"cr={f['cr_vs_oracle']:.2f}%")
        if "cr_dev_vs_exact" in f:
            line += (f" | exact: cr {f['cr_dev_vs_exact']:.2f}/{f['cr_oracle_vs_exact']:.2f}/"
                     f"{f['cr_need']:.2f}% err mean {f['err_dev_mean']:.2e}/{f['err_oracle_mean']:.2e}"
                     f" max {f['err_dev_max']:.2e}/{f['err_oracle_max']:.2e}")
        tr.write_line(line)
