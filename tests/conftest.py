import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def oracle():
    from tests.support.oracle_lib import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def reference():
    """The reference's own code, compiled from /root/reference into oracle/_ref.
    Absent where it was not built (the GPU box has no /root/reference)."""
    from tests.support.oracle_lib import reference_or_none

    ref = reference_or_none()
    if ref is None:
        pytest.skip("oracle/_ref is not built here (needs /root/reference)")
    return ref


@pytest.fixture(scope="session")
def fixture_tensors():
    from tests.support import gguf_fixture

    return gguf_fixture.read(os.path.join(ROOT, "tests", "golden", "matmul_rows.gguf"))
