import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "velo-core_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP code object")


@pytest.fixture(scope="session")
def ctx():
    """The one HIP context of the GPU test session. Fails (does not skip) when the
    device or the code object is missing: GPU tests never fall back to the CPU."""
    import velokv
    c = velokv.Context(0)
    yield c
    c.close()
