import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def hip():
    """The HIP C ABI.  GPU tests fail loudly if the library or the GPU is missing."""
    from ml_engine_amd import hip as h

    h.init(0)
    return h


@pytest.fixture(scope="session")
def orc():
    import oracle_lib

    oracle_lib.lib()
    return oracle_lib


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def assert_close(got: np.ndarray, ref: np.ndarray, rtol: float, atol_scale: float = 0.0, what: str = "",
                 scale: float | None = None):
    """|got - ref| <= rtol*|ref| + atol_scale*S element-wise, S = max|ref| or `scale`.

    The absolute floor is relative to the magnitude of the summed terms: GEMM
    and reduction outputs near zero carry cancellation error of that size, not
    of the result.  A result that is zero by symmetry (for example a bias
    gradient whose row sums cancel exactly) passes the magnitude of its terms
    as `scale`.
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if ref.size == 0:
        return
    assert np.all(np.isfinite(got) == np.isfinite(ref)), f"{what}: finiteness differs"
    fin = np.isfinite(ref)
    if scale is None:
        scale = np.max(np.abs(ref[fin])) if fin.any() else 0.0
    err = np.abs(got - ref)
    tol = rtol * np.abs(ref) + atol_scale * scale
    bad = fin & (err > tol)
    if bad.any():
        i = np.argmax(np.where(bad, err - tol, -np.inf))
        idx = np.unravel_index(i, ref.shape)
        raise AssertionError(
            f"{what}: {bad.sum()} / {ref.size} elements out of tolerance (rtol {rtol}, atol {atol_scale}*{scale:.3g}); "
            f"worst at {idx}: got {got[idx]!r} ref {ref[idx]!r} err {err[idx]:.3g}"
        )
