"""pytest configuration: the ``gpu`` marker, import paths and shared fixtures.

``-m "not gpu"`` runs the oracle pins, host logic and C-ABI validation on the CPU;
``-m gpu`` runs the HIP parity tests on an MI355X (they are skipped when no GPU is visible).
"""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

# @pytest.mark.metrics, --csv-output and --iterations (the reference harness's metrics CSV)
pytest_plugins = ["iron_amd.common.test_metrics"]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running (full-model) test")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle_provider():
    """Install the CPU oracle as the source of ``op.reference()`` for the session."""
    from iron_amd.common.base import register_reference_provider
    from oracle.provider import reference

    register_reference_provider(reference)
    yield reference
    register_reference_provider(None)


@pytest.fixture(scope="session")
def lib():
    from iron_amd import _lib

    return _lib.load()


def pytest_report_header(config):
    return f"iron_amd tests (HIP library: {REPO / 'iron_amd' / 'libiron_hip.so'})"
