import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def pytest_collection_modifyitems(config, items):
    # Fail loudly instead of skipping: a gpu-marked test on a box without a GPU
    # or without the built library must not pass silently.
    pass


@pytest.fixture(scope="session")
def oracle():
    from oracle import load_oracle
    return load_oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import load_ref
    r = load_ref()
    if r is None:
        pytest.skip("oracle/_ref (compiled reference) not built here")
    return r
