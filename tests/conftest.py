import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, GOLDEN)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle
    return Oracle(threads=min(os.cpu_count() or 1, 16))


@pytest.fixture(scope="session")
def ref():
    from oracle import Ref, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref/libref.so not built (reference sources absent)")
    return Ref(threads=min(os.cpu_count() or 1, 8))


@pytest.fixture(scope="session")
def ctx():
    import guanaco_amd.hip as H
    c = H.Context(0)  # raises loudly when no GPU / library: GPU tests must not silently pass
    yield c
    c.close()
