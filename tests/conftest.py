# SPDX-License-Identifier: MPL-2.0
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):  # bmhip (the ctypes wrapper) and the oracle
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


@pytest.fixture(scope="session")
def be():
    """One HIP backend context for every GPU test in the session."""
    import bmhip

    b = bmhip.Backend()
    yield b
    b.close()
