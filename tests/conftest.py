import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("irodori-c_amd", "oracle"):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


_CTX = {}


def _ctx(conv):
    import iro_hip
    if conv not in _CTX:
        _CTX[conv] = iro_hip.Context(0, conv)
    return _CTX[conv]


@pytest.fixture(scope="session")
def ctx_strict():
    return _ctx(0)


@pytest.fixture(scope="session")
def ctx_fast():
    return _ctx(1)


@pytest.fixture(scope="session", params=[0, 1], ids=["strict", "fastmath"])
def ctx(request):
    return _ctx(request.param)


@pytest.fixture(autouse=True)
def _release_device_memory():
    yield
    for c in _CTX.values():
        c.release_all()


def pytest_sessionfinish(session, exitstatus):
    for c in _CTX.values():
        c.close()
    _CTX.clear()
