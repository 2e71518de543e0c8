import gc
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libxlog_hip.so on cuda:0)")


@pytest.fixture(scope="session")
def provider():
    from xlog_amd import HipKernelProvider

    p = HipKernelProvider(0)
    yield p
    p.close()


@pytest.fixture(autouse=True)
def _release_device_relations():
    """Relation handles free their device memory when collected.  A test whose
    frame holds a pytest.raises result is in a reference cycle (frame ->
    exception -> traceback -> frame) that only the cycle collector breaks, so
    its relations would stay live into later tests: collect after each test."""
    yield
    gc.collect()
