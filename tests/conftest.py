"""Test configuration.

``-m gpu`` tests need the gfx950 library and a GPU; everything else runs on
the CPU (oracle pins, format known-answer tests, ABI symbol checks).
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def gpu_present() -> bool:
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def ref_available():
    import oracle
    return oracle.ref() is not None
