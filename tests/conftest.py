import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs through the HIP C-ABI)")


@pytest.fixture(scope="session")
def oracle():
    from oracle_ffi import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle_ffi import load_ref
    lib = load_ref()
    if lib is None:
        pytest.skip("oracle/_ref not built (reference tree absent and no prebuilt copy)")
    return lib
