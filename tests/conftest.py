import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "tmac_gguf.cpp_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# Parity rule for fp32 outputs:
#   |gpu - ref| <= ATOL + RTOL * |ref| elementwise.
ATOL = 2e-5
RTOL = 1e-4


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def assert_close(got, ref, what="", atol=ATOL, rtol=RTOL):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    tol = atol + rtol * np.abs(ref)
    bad = ~(err <= tol)
    if bad.any():
        i = int(np.flatnonzero(bad.ravel())[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} elements outside {atol}+{rtol}|ref|; "
            f"max_abs={err.max():.3e}; first bad flat index {i}: got {got.ravel()[i]!r} ref {ref.ravel()[i]!r}")
    return float(err.max()) if err.size else 0.0


@pytest.fixture(scope="session")
def ctx():
    import tmac_attn

    c = tmac_attn.Context(0)
    yield c
    c.close()
