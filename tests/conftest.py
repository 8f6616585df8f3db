import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "flat-attention_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def assert_close(name, actual, expected, atol, rtol):
    """|a - e| <= atol + rtol*|e| elementwise (the reference tests' assert_close)."""
    actual = np.asarray(actual, np.float64).ravel()
    expected = np.asarray(expected, np.float64).ravel()
    assert actual.shape == expected.shape, f"{name}: shape {actual.shape} vs {expected.shape}"
    assert np.all(np.isfinite(actual)), f"{name}: non-finite output"
    err = np.abs(actual - expected)
    tol = atol + rtol * np.abs(expected)
    bad = np.nonzero(err > tol)[0]
    if bad.size:
        i = bad[np.argmax(err[bad] - tol[bad])]
        raise AssertionError(
            f"{name}: {bad.size} of {actual.size} outside tolerance; worst index {i}: "
            f"actual={actual[i]!r} expected={expected[i]!r} err={err[i]:.3e} tol={tol[i]:.3e} "
            f"(max abs err {err.max():.3e})")


@pytest.fixture(scope="session")
def hip():
    """Session-wide HIP context on cuda:0 (gpu tests only). Fails loudly without the library."""
    import flat_attention_amd as fa
    ctx = fa.HipContext(0)
    yield ctx
    ctx.close()
