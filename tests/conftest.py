"""Pytest configuration: markers and import path.

``gpu``  — needs an MI355X; the round-end GPU run selects these with ``-m gpu``.
``slow`` — large CPU oracle work; skipped unless ``--runslow`` is given
           (mirrors the reference's conftest.py:11-32).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_addoption(parser):
    parser.addoption("--runslow", action="store_true", default=False,
                     help="run slow cases (large CPU oracle work)")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950)")
    config.addinivalue_line("markers", "slow: large case; skipped unless --runslow")


def pytest_collection_modifyitems(config, items):
    if config.getoption("--runslow"):
        return
    skip = pytest.mark.skip(reason="slow case; pass --runslow to run")
    for item in items:
        if "slow" in item.keywords:
            item.add_marker(skip)
