import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure), built on first use."""
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def kern():
    """The product's host API; on a GPU box it must load libgrx.so and see a GPU."""
    from gorelaxor_amd import kern as k

    if k.device_count() < 1:
        pytest.fail("no GPU visible: the gpu tests need an MI355X")
    return k
