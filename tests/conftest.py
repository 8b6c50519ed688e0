import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def golden():
    """Load a golden .npz by name (files written by tests/golden/make_golden.py)."""
    manifest = json.load(open(os.path.join(GOLDEN, "MANIFEST.json")))

    def load(name):
        assert name in manifest, name
        return np.load(os.path.join(GOLDEN, name), allow_pickle=False)

    return load


@pytest.fixture(scope="session")
def rocm():
    """The product's C-ABI library (GPU tests only)."""
    from pyflamert_amd import _lib

    return _lib.load()
