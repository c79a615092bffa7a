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
def torch_cuda():
    """torch with a usable GPU (device memory and streams only)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test without a GPU: run with -m 'not gpu' on a CPU host")
    return torch


@pytest.fixture(scope="session")
def kernels(torch_cuda):
    from decide_amd.kernels import Kernels

    k = Kernels()
    yield k
    k.ctx.close()


@pytest.fixture(scope="session")
def kernels_ref(torch_cuda):
    from decide_amd.kernels import GemmImpl, Kernels

    k = Kernels(GemmImpl.Baseline)
    yield k
    k.ctx.close()


@pytest.fixture()
def stream(torch_cuda):
    return torch_cuda.cuda.current_stream().cuda_stream
