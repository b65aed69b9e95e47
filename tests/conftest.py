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
