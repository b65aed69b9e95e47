"""pytest configuration: the ``gpu`` marker, import paths and the per-case
parity figures printed at the end of a session.

GPU tests carry ``@pytest.mark.gpu``; the CPU suite runs with ``-m "not gpu"``.
The full-size cases (the 128 x 131072 decode and the 8192-token prefill) run by
default: the oracle finishes them in seconds, so there is no slow gate.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


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
