import os
import sys

import numpy as np
import pytest

# torch ships its own HIP runtime under the same SONAME (libamdhip64.so.7)
# as /opt/rocm's; whichever is loaded first serves the whole process.  Tests
# that hand torch device buffers to libtomoul_hip need torch's copy loaded
# before the library, so import torch first when it is installed.
try:
    import torch  # noqa: F401
except ImportError:  # pragma: no cover
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libtomoul_hip.so")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (built on first use)."""
    from oracle import oracle as o
    o.lib()
    return o


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max|G - R| / max|R| (infinity-norm relative error)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref)) if ref.size else 0.0
    if denom == 0.0:
        return float(np.max(np.abs(got))) if got.size else 0.0
    return float(np.max(np.abs(got - ref)) / denom)


def elementwise_ok(got: np.ndarray, ref: np.ndarray, tol: float) -> bool:
    """|G - R| <= tol * (|R| + rms(R)) for every element."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return True
    rms = float(np.sqrt(np.mean(ref * ref)))
    return bool(np.all(np.abs(got - ref) <= tol * (np.abs(ref) + rms) + 1e-30))
