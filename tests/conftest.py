import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def assert_close(actual, expected, abs_tol=1e-4, rel_tol=1e-5):
    """The reference's mixed tolerance (backend-cpu/src/reference/mod.rs:154-165):
    an element passes when |a - e| <= max(abs_tol, rel_tol * |e|)."""
    import numpy as np

    actual = np.asarray(actual, dtype=np.float64).ravel()
    expected = np.asarray(expected, dtype=np.float64).ravel()
    assert actual.shape == expected.shape, "output length mismatch"
    diff = np.abs(actual - expected)
    tol = np.maximum(abs_tol, rel_tol * np.abs(expected))
    bad = np.nonzero(~(diff <= tol))[0]
    assert bad.size == 0, (
        f"mismatch at index {bad[0]}: actual={actual[bad[0]]}, expected={expected[bad[0]]}, "
        f"difference={diff[bad[0]]}, tolerance={tol[bad[0]]}"
    )


@pytest.fixture(scope="session", autouse=True)
def _oracle_threads():
    """The oracle spreads independent outputs over up to 16 threads in the
    tests (bit-identical to one thread; tests/test_oracle_threads.py)."""
    import oracle as o

    o.lib()
    o.set_threads(min(16, os.cpu_count() or 1))
    yield


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


def rel_l2(actual, expected):
    """Normwise relative error ||a - e||_2 / ||e||_2 (0 when both are zero)."""
    import numpy as np

    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    assert a.shape == e.shape, f"shape mismatch {a.shape} vs {e.shape}"
    den = np.linalg.norm(e)
    num = np.linalg.norm(a - e)
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return float(num / den)


# Tolerances of the GPU-vs-oracle comparisons.
ELEMENTWISE_REL = 1e-6   # per element, fp32 elementwise ops
NORMWISE_REL = 1e-4      # ||gpu - cpu||_2 / ||cpu||_2 for reductions, matmul, attention


def assert_elementwise(actual, expected, rel=ELEMENTWISE_REL):
    import numpy as np

    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    assert a.shape == e.shape
    bad = np.nonzero(np.abs(a - e) > rel * np.abs(e) + 1e-30)[0]
    assert bad.size == 0, f"index {bad[0]}: {a[bad[0]]!r} vs {e[bad[0]]!r}"


def assert_normwise(actual, expected, rel=NORMWISE_REL):
    err = rel_l2(actual, expected)
    assert err <= rel, f"normwise relative error {err:.3e} > {rel:.0e}"


@pytest.fixture(scope="session")
def hip():
    """The GPU device under test (only for tests marked gpu)."""
    from starlight_amd.device import HipDevice

    dev = HipDevice(0)
    yield dev
    dev.close()
