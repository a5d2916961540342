import os
import sys

import pytest

try:  # load torch's HIP runtime first, as bench.py does, so one runtime serves both
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    from bind import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from bind import Ref
    if not Ref.available:
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    return Ref()
