import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C-ABI")


@pytest.fixture(scope="session")
def oracle():
    from oracle.binding import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref_scalar():
    from oracle.binding import Ref
    if not Ref.available(scalar=True):
        pytest.skip("oracle/_ref not built (needs the reference sources; `make -C oracle ref`)")
    return Ref(scalar=True)


@pytest.fixture(scope="session")
def ref_avx2():
    from oracle.binding import Ref
    if not Ref.available(scalar=False):
        pytest.skip("oracle/_ref not built (needs the reference sources; `make -C oracle ref`)")
    return Ref(scalar=False)
