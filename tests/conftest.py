import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture
def rng():
    return np.random.default_rng(12345)


@pytest.fixture(scope="session")
def ref():
    """The compiled reference (oracle/_ref), bound with the shared signature table."""
    import oracle
    from acfun_amd.capi import bind
    r = oracle.ref()
    if r is None:
        pytest.skip("oracle/_ref/libacfun_ref.so not built (needs /root/reference): make -C oracle")
    return bind(r)


@pytest.fixture(scope="session")
def olib():
    import oracle
    return oracle.lib()


@pytest.fixture(scope="session")
def gpu():
    """The product library on a GPU; GPU tests fail (not skip) if it is unusable."""
    from acfun_amd import capi
    L = capi.lib()
    if L.acfun_backend() != 4:
        pytest.fail("no usable gfx950 device: " + capi.last_error())
    return L
