import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def cpuref():
    import oracle
    if not os.path.exists(oracle.CPUREF_SO):
        oracle.build(with_ref=False)
    return oracle.CpuRef()


@pytest.fixture(scope="session")
def refc():
    """The reference engine itself (oracle/_ref), when it was built."""
    import oracle
    if not oracle.have_ref():
        pytest.skip("oracle/_ref/libref.so not built (reference sources absent at build time)")
    return oracle.Ref()


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="session")
def ctx(torch_gpu):
    import llama3pure_amd as l3p
    torch_gpu.cuda.init()
    c = l3p.Context(0)
    yield c
    c.close()


def f32_bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)
