import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mythos.cpp_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def mth():
    import mythos_oil
    return mythos_oil


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU")
    return torch.device("cuda:0")


def fp32_close(got, ref, absw, rel=1e-5, what=""):
    """Norm-wise ||got-ref|| <= rel*||ref|| and element-wise
    |got-ref| <= rel*sum_k|w_k x_k| (+ a denormal floor): the FP32 tolerance
    for reordered summation, robust to cancellation."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    absw = np.asarray(absw, np.float64).ravel()
    d = np.abs(got - ref)
    nrm = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    bad = d > rel * absw + 1e-30
    assert nrm <= rel, f"{what}: norm-wise rel err {nrm:.3e} > {rel}"
    assert not bad.any(), (f"{what}: {bad.sum()} elements exceed {rel}*sum|wx|; "
                           f"worst {d[bad].max():.3e} vs bound {(rel * absw[bad]).min():.3e}")
    return nrm
