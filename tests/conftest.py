import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.pyoracle import Oracle, build
    build()
    return Oracle()


@pytest.fixture(scope="session")
def be():
    from shiftwing_amd import Backend
    return Backend(0)


def rms(a):
    a = np.asarray(a, np.float64)
    return float(np.sqrt(np.mean(a * a)))


def assert_close_rms(got, want, tol=1e-3, what=""):
    """The north-star tolerance: max |got - want| <= tol * RMS(want)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    bound = tol * rms(want)
    assert err <= bound, f"{what}: max abs err {err:.3e} > {tol} x RMS {rms(want):.3e}"
    return err / max(rms(want), 1e-30)
