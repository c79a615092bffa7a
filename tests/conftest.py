import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """A usable GPU, reached through the HIP runtime libdecide_hip.so links (no torch)."""
    from decide_amd import hip

    if not hip.available():
        pytest.fail("gpu test without a GPU: run with -m 'not gpu' on a CPU host")
    return hip


@pytest.fixture(scope="session")
def kernels(gpu):
    from decide_amd.kernels import Kernels

    k = Kernels()
    yield k
    k.ctx.close()


@pytest.fixture(scope="session")
def kernels_ref(gpu):
    from decide_amd.kernels import GemmImpl, Kernels

    k = Kernels(GemmImpl.Baseline)
    yield k
    k.ctx.close()


@pytest.fixture()
def stream(gpu):
    """The legacy default stream (0): synchronous copies order against it."""
    return 0


@pytest.fixture(scope="session")
def kernels_delta_chunked(gpu):
    """A context whose gated delta always runs the chunked recurrence."""
    from decide_amd.kernels import Kernels

    k = Kernels(delta="chunked")
    yield k
    k.ctx.close()


@pytest.fixture(scope="session")
def kernels_delta_sequential(gpu):
    """A context whose gated delta always runs the token-by-token kernel."""
    from decide_amd.kernels import Kernels

    k = Kernels(delta="sequential")
    yield k
    k.ctx.close()
