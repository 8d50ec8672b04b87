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


def is_half_nan(h: np.ndarray, dt: int) -> np.ndarray:
    """NaN patterns of f16 (dt 0) or bf16 (dt 1) bits."""
    h = np.asarray(h).astype(np.uint32)
    if dt == 0:
        return ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    return ((h & 0x7F80) == 0x7F80) & ((h & 0x7F) != 0)


def half_nan_candidates(orc, ha: np.ndarray, hb: np.ndarray, dt: int):
    """The admissible results of NaN op NaN on the half path: either operand's
    NaN, decoded to f32, quieted (bit 22 set, sign and payload kept) and
    encoded again. Which of the two survives follows the compiler's operand
    order on the reference's side, so nothing narrower is pinned."""
    def quieted(h):
        f = orc.decode_half(np.ascontiguousarray(h, np.uint16), dt).view(np.uint32)
        return orc.encode_half((f | np.uint32(0x00400000)).view(np.float32), dt)
    return quieted(ha), quieted(hb)


def assert_half_result(orc, got, want, ha, hb, dt, what: str = "") -> int:
    """Bit-exact against `want` wherever at least one operand is not NaN; where
    both are NaN, one of the two admissible quieted payloads. Returns the
    number of NaN-op-NaN elements checked that way."""
    got, want = np.asarray(got).reshape(-1), np.asarray(want).reshape(-1)
    ha, hb = np.asarray(ha).reshape(-1), np.asarray(hb).reshape(-1)
    both = is_half_nan(ha, dt) & is_half_nan(hb, dt)
    assert_bitexact(got[~both], want[~both], what)
    if both.any():
        ca, cb = half_nan_candidates(orc, ha[both], hb[both], dt)
        g = got[both]
        bad = np.nonzero((g != ca) & (g != cb))[0]
        if len(bad):
            i = int(bad[0])
            raise AssertionError(
                f"{what}: NaN op NaN gave {int(g[i]):#06x}, admissible {int(ca[i]):#06x} "
                f"or {int(cb[i]):#06x} ({len(bad)} of {g.size} outside the set)")
    return int(both.sum())
