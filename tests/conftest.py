import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "agention-infer_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def backend():
    import gq
    be = gq.create_backend("hip")
    # IQ3_XXS weights need a codebook installed first: the synthetic
    # weights of the tests use the library's built-in test codebook (the
    # oracle's default table).
    be.set_iq3xxs_grid(None)
    return be
