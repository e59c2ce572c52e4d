"""Shared pytest configuration: the `gpu` marker and lazily built test
libraries (the oracle is test infrastructure; the product library is built by
__graft_entry__.build())."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.pyoracle import ORACLE_SO, Oracle, build
    if not os.path.exists(ORACLE_SO):
        build()
    return Oracle()


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    gdir = os.path.join(ROOT, "tests", "golden")

    def load(name):
        with np.load(os.path.join(gdir, name)) as z:
            return {k: z[k] for k in z.files}

    return load
