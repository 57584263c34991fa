"""Test configuration. `-m gpu` tests need an MI355X and call the HIP library
through its C ABI; everything else runs on the CPU (oracle against golden
vectors, host logic, library exports)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

REFERENCE = "/root/reference"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built HIP library")


def tol_ok(actual, expected, abs_tol=1e-4, rel_tol=1e-3):
    """|a - e| <= abs_tol + rel_tol * |e| element-wise (layer-output tolerance)."""
    import numpy as np
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return bool(np.all(np.isfinite(a)) and np.all(np.abs(a - e) <= abs_tol + rel_tol * np.abs(e)))


# Batches of this many tokens or more route with the certified batch router.
CERTIFIED_MIN_TOKENS = 512


def weights_close(actual, expected, rel_tol=1e-6):
    """Routing weights of the certified batch router: its sum of
    exponentials uses approximate logits for the experts that are not near
    the top-k boundary, so a weight may differ from the reference's by a few
    ulp; |a - e| <= rel_tol |e| element-wise."""
    import numpy as np
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return bool(a.shape == e.shape and np.all(np.isfinite(a)) and np.all(np.abs(a - e) <= rel_tol * np.abs(e)))


def weights_ok(tokens, actual, expected):
    """Bit-exact below CERTIFIED_MIN_TOKENS (the exact routers), within
    1e-6 relative from there on (the certified router)."""
    import numpy as np
    if tokens < CERTIFIED_MIN_TOKENS:
        return np.array_equal(np.asarray(actual, np.float32).view(np.uint32),
                              np.asarray(expected, np.float32).view(np.uint32))
    return weights_close(actual, expected)


def ref_compare(actual, expected, tol=2e-5):
    """The reference's own comparison rule |a - e| <= tol * (1 + |e|)
    (tests/conformance.js:7-10); returns the max absolute error."""
    import numpy as np
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, "length mismatch"
    err = np.abs(a - e)
    bad = ~np.isfinite(a) | (err > tol * (1 + np.abs(e)))
    assert not bad.any(), "values[%d]: %r versus %r" % (int(np.argmax(bad)), a[bad][0], e[bad][0])
    return float(err.max()) if err.size else 0.0


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def backend():
    import stratacuda_amd as sm
    b = sm.Backend(0)
    yield b
    b.dispose()
