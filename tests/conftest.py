import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "splatx-metal_amd", "python"), os.path.join(REPO, "oracle"),
          os.path.join(REPO, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import oracle_py
    return oracle_py.Oracle(libm=False)


@pytest.fixture(scope="session")
def oracle_libm():
    import oracle_py
    return oracle_py.Oracle(libm=True)


@pytest.fixture(scope="session", params=["sx", "libm"])
def any_oracle(request):
    import oracle_py
    return oracle_py.Oracle(libm=(request.param == "libm"))


@pytest.fixture(scope="session")
def reference():
    import oracle_py
    if not oracle_py.Reference.available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return oracle_py.Reference()


@pytest.fixture(scope="session")
def gpu():
    import splatx_hip
    b = splatx_hip.Backend(0)
    yield b
    b.close()
