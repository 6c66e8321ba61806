import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "suzuku-engine-q4_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as om
    return om.Oracle()


@pytest.fixture(scope="session")
def ref():
    import oracle as om
    if not om.have_ref():
        pytest.skip("reference build oracle/_ref not present")
    return om.Ref()


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0, launching on torch's current stream."""
    import torch
    import q4mi
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    L = q4mi.lib()
    assert L.q4mi_device_ok()
    q4mi.use_torch_stream()
    return L


@pytest.fixture(scope="session")
def gpu_meas(gpu):
    """The measurement build (product ABI + include/q4mi_measure.h hooks) on
    the same stream."""
    import q4mi
    M = q4mi.meas()
    assert M.q4mi_device_ok()
    q4mi.use_torch_stream(M)
    return M


def layer_err(got, ref):
    """max |got-ref| / max|ref| (normwise)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def rel_err(got, ref):
    """max |got-ref| / max(|ref|, 1e-3 * max|ref|): elementwise relative error
    with values near zero measured against 1e-3 of the output's scale."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = 1e-3 * max(np.abs(ref).max(), 1e-30)
    return float((np.abs(got - ref) / np.maximum(np.abs(ref), floor)).max())
