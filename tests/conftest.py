"""Shared fixtures. `gpu` tests need a real MI355X and the built library;
everything else runs on any host (the oracle, the ABI surface, host logic)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "magnetar-provider-cuda_amd")
for path in (ROOT, PKG):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libmagnetar_hip.so")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import magnetar_hip
    device = magnetar_hip.Device(0)
    yield device
    device.close()


def bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a.view(np.uint16)


def assert_bitexact(actual: np.ndarray, expected: np.ndarray, what: str = ""):
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    ab, eb = bits(actual).reshape(-1), bits(expected).reshape(-1)
    bad = np.nonzero(ab != eb)[0]
    if len(bad):
        i = int(bad[0])
        raise AssertionError(
            f"{what}: {len(bad)} of {ab.size} differ; first at flat index {i}: "
            f"{actual.reshape(-1)[i]!r} ({ab[i]:#x}) vs {expected.reshape(-1)[i]!r} ({eb[i]:#x})")


def max_rel_err(actual, expected, floor: float = 1e-30) -> float:
    """max_i |a_i - e_i| / max(|e_i|, floor) (elementwise relative error)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return float(np.max(np.abs(a - e) / np.maximum(np.abs(e), floor))) if a.size else 0.0


def max_normwise_err(actual, expected) -> float:
    """max_i |a_i - e_i| / max_i |e_i| (error relative to the tensor's largest entry)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    if a.size == 0:
        return 0.0
    scale = float(np.max(np.abs(e)))
    return float(np.max(np.abs(a - e))) / (scale if scale > 0 else 1.0)


def max_rel_err_significant(actual, expected, frac: float = 1e-3) -> float:
    """max_i |a_i - e_i| / |e_i| over the entries with |e_i| >= frac * max|e|:
    the elementwise relative error where it is defined (an entry that cancels
    to ~0 has none)."""
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    if a.size == 0:
        return 0.0
    keep = np.abs(e) >= frac * float(np.max(np.abs(e)))
    if not keep.any():
        return 0.0
    return float(np.max(np.abs(a[keep] - e[keep]) / np.abs(e[keep])))


def sweep_seeds(n: int) -> range:
    """Seeds of a randomized sweep: n by default, n * MHIP_SWEEP_SCALE when
    that is set (a wider sweep on demand; every seed is its own case)."""
    import os
    return range(n * max(1, int(os.environ.get("MHIP_SWEEP_SCALE", "1"))))
