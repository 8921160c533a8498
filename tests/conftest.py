import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE / "golden"))
sys.path.insert(0, str(HERE.parent / "oracle"))
sys.path.insert(0, str(HERE.parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle_bind
    return oracle_bind


@pytest.fixture(scope="session")
def ref_lib():
    import oracle_bind
    r = oracle_bind.ref()
    if r is None:
        pytest.skip("oracle/_ref/libpairef.so not built (reference tree absent at build time)")
    return r
