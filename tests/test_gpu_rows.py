"""GPU parity: RMSNorm, row softmax and RoPE against the CPU oracle.

Bars (north star): rmsnorm and softmax within 1e-4 max relative error
(elementwise, |gpu - cpu| / |cpu|); rope, an elementwise op, within 1e-6 of
each rotated pair's magnitude (|gpu - cpu| / sqrt(a^2 + b^2)) -- a rotation's
outputs can cancel to near zero, where a relative bar on the output itself
measures sin/cos rounding in the input's units rather than an error. The
measured errors are printed so each kernel's error is on record.
"""
import numpy as np
import pytest

from conftest import assert_bitexact, max_rel_err

pytestmark = pytest.mark.gpu

RMS_TOL = 1e-4
SOFTMAX_TOL = 1e-4
ROPE_TOL = 1e-6


# ---- rmsnorm ------------------------------------------------------------------

def test_rmsnorm_reference_fixture(dev, orc):
    """src/tests_conformance.rs:177-189."""
    from magnetar_hip import ops
    x = np.array([1.0, 2.0, 3.0, -1.0, 0.5, 2.0], np.float32).reshape(2, 3)
    w = np.array([1.0, 0.5, 2.0], np.float32)
    got = ops.rmsnorm(dev, dev.upload(x), dev.upload(w), 1e-5).numpy()
    assert max_rel_err(got, orc.rmsnorm(x, w, 1e-5)[0]) <= RMS_TOL


@pytest.mark.parametrize("rows,cols", [(1, 4), (5, 3), (32, 256), (3, 64), (17, 1000),
                                       (9, 1024), (4, 2048), (16, 4096), (2, 4100),
                                       (3, 11008), (2, 16384), (2, 20000), (1, 7)])
@pytest.mark.parametrize("weight_mode", ["row", "none", "per_row"])
def test_rmsnorm_shapes(dev, orc, rows, cols, weight_mode):
    from magnetar_hip import ops
    x = orc.normal(rows * cols, 41).reshape(rows, cols)
    if weight_mode == "row":
        w, stride = orc.normal(cols, 42, 1.0, 0.1), 0
    elif weight_mode == "per_row":
        w, stride = orc.normal(rows * cols, 43, 1.0, 0.1).reshape(rows, cols), cols
    else:
        w, stride = None, 0
    got = ops.rmsnorm(dev, dev.upload(x), dev.upload(w) if w is not None else None, 1e-5,
                      weight_row_stride=stride).numpy()
    want, st = orc.rmsnorm(x, w, 1e-5, weight_row_stride=stride)
    assert st == 0
    err = max_rel_err(got, want)
    print(f"rmsnorm [{rows},{cols}] {weight_mode}: max rel err {err:.3e}")
    assert err <= RMS_TOL


@pytest.mark.parametrize("rows,cols,gain", [(2048, 4096, True), (2049, 4096, False),
                                            (1031, 3000, True), (1100, 2052, True)])
def test_rmsnorm_many_rows_match_small_batches(dev, orc, rows, cols, gain):
    """From 1024 rows of 513-1024 vectors on, RMSNorm runs a 1024-thread
    kernel that takes two rows per workgroup (odd row counts and partial
    last chunks clamp to the last row and column). Its bits must equal the
    one-row-per-workgroup kernel's, which batches of fewer rows still take,
    and the oracle within the bar."""
    from magnetar_hip import ops
    x = orc.normal(rows * cols, 46).reshape(rows, cols)
    w = orc.normal(cols, 47, 1.0, 0.1) if gain else None
    dw = dev.upload(w) if gain else None
    whole = ops.rmsnorm(dev, dev.upload(x), dw, 1e-5).numpy()
    for r0 in range(0, rows, 500):
        part = ops.rmsnorm(dev, dev.upload(np.ascontiguousarray(x[r0:r0 + 500])), dw, 1e-5).numpy()
        assert_bitexact(whole[r0:r0 + 500], part)
    want, st = orc.rmsnorm(x, w, 1e-5)
    assert st == 0
    assert max_rel_err(whole, want) <= RMS_TOL


def test_rmsnorm_per_head(dev, orc):
    """Per-head normalisation: rows of [rows * heads, head_dim] (src/kernels.rs:4013-4040)."""
    from magnetar_hip import ops
    rows, heads, hd = 7, 4, 64
    x = orc.normal(rows * heads * hd, 44).reshape(rows, heads * hd)
    w = orc.normal(hd, 45, 1.0, 0.1)
    got = ops.rmsnorm(dev, dev.upload(x), dev.upload(w), 1e-6, cols=hd).numpy()
    want, st = orc.rmsnorm(x, w, 1e-6, cols=hd)
    assert max_rel_err(got, want) <= RMS_TOL


def test_rmsnorm_rejects_bad_epsilon(dev):
    from magnetar_hip import ops, MagnetarHipError
    x = dev.upload(np.ones((2, 4), np.float32))
    with pytest.raises(MagnetarHipError) as err:
        ops.rmsnorm(dev, x, None, 0.0)
    assert err.value.code == "ShapeUnsupported"


def test_rmsnorm_baseline_shape(dev, orc):
    """[8192, 4096], gain ~N(1, 0.1), eps 1e-5."""
    from magnetar_hip import ops
    x = orc.normal(8192 * 4096, 51).reshape(8192, 4096)
    w = orc.normal(4096, 52, 1.0, 0.1)
    got = ops.rmsnorm(dev, dev.upload(x), dev.upload(w), 1e-5).numpy()
    err = max_rel_err(got, orc.rmsnorm(x, w, 1e-5)[0])
    print(f"rmsnorm [8192,4096]: max rel err {err:.3e}")
    assert err <= RMS_TOL


# ---- softmax ------------------------------------------------------------------

def test_softmax_reference_fixture(dev, orc):
    """src/tests_conformance.rs:127-136."""
    from magnetar_hip import ops
    x = np.array([1.0, 2.0, 3.0, -1.0, 0.0, 1.0], np.float32).reshape(2, 3)
    got = ops.softmax_rows(dev, dev.upload(x)).numpy()
    assert dev.check_flags() == 0
    assert max_rel_err(got, orc.softmax_rows(x)[0]) <= SOFTMAX_TOL


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 3), (32, 32), (8, 256), (17, 1000),
                                       (9, 1024), (4, 2048), (16, 4096), (2, 4100),
                                       (3, 16384), (2, 30000)])
def test_softmax_shapes(dev, orc, rows, cols):
    from magnetar_hip import ops
    x = orc.normal(rows * cols, 61, 0.0, 2.0).reshape(rows, cols)
    got = ops.softmax_rows(dev, dev.upload(x)).numpy()
    assert dev.check_flags() == 0
    want, st = orc.softmax_rows(x)
    assert st == 0
    err = max_rel_err(got, want)
    print(f"softmax [{rows},{cols}]: max rel err {err:.3e}")
    assert err <= SOFTMAX_TOL


def test_softmax_masked_entries_and_failure(dev, orc):
    from magnetar_hip import ops, MagnetarHipError
    x = np.array([[0.0, -np.inf, 1.0, -np.inf], [2.0, 2.0, 2.0, 2.0]], np.float32)
    got = ops.softmax_rows(dev, dev.upload(x)).numpy()
    assert dev.check_flags() == 0
    assert got[0, 1] == 0.0 and got[0, 3] == 0.0
    assert max_rel_err(got, orc.softmax_rows(x)[0]) <= SOFTMAX_TOL
    bad = np.array([[0.0, 1.0], [-np.inf, -np.inf]], np.float32)
    assert orc.softmax_rows(bad)[1] == 4
    ops.softmax_rows(dev, dev.upload(bad))
    with pytest.raises(MagnetarHipError) as err:
        dev.check_flags()
    assert err.value.code == "ExecutionFailed"
    # A NaN entry is ignored by the max (fmaxf), so the row does not fail.
    nan_row = np.array([[np.nan, 1.0, 2.0, 3.0]], np.float32)
    ops.softmax_rows(dev, dev.upload(nan_row))
    assert dev.check_flags() == 0


def test_softmax_baseline_shape(dev, orc):
    """[8192, 4096] ~N(0, 4)."""
    from magnetar_hip import ops
    x = orc.normal(8192 * 4096, 62, 0.0, 2.0).reshape(8192, 4096)
    got = ops.softmax_rows(dev, dev.upload(x)).numpy()
    assert dev.check_flags() == 0
    err = max_rel_err(got, orc.softmax_rows(x)[0])
    print(f"softmax [8192,4096]: max rel err {err:.3e}")
    assert err <= SOFTMAX_TOL


# ---- rope ---------------------------------------------------------------------

def rope_pair_err(x, got, want, params):
    """max |got - want| / |(a, b)| over every element of every rotated pair."""
    rows, cols = x.shape
    hw = cols // params.head_count
    half = params.dimension // 2
    x = x.astype(np.float64).reshape(rows, params.head_count, hw)
    g = got.astype(np.float64).reshape(rows, params.head_count, hw)
    w = want.astype(np.float64).reshape(rows, params.head_count, hw)
    p = np.arange(half)
    i1 = p if params.half_split else 2 * p
    i2 = p + half if params.half_split else 2 * p + 1
    norm = np.sqrt(x[..., i1] ** 2 + x[..., i2] ** 2)
    norm = np.maximum(norm, 1e-30)
    e1 = np.abs(g[..., i1] - w[..., i1]) / norm
    e2 = np.abs(g[..., i2] - w[..., i2]) / norm
    rest = np.setdiff1d(np.arange(hw), np.concatenate([i1, i2]))
    assert np.array_equal(g[..., rest], x[..., rest]), "pass-through columns changed"
    return float(max(e1.max(initial=0), e2.max(initial=0)))


ROPE_CASES = [
    # (rows, cols, dimension, offset, heads, half_split) -- the reference's fixtures first
    (2, 4, 4, 0, 1, 0),       # src/tests_conformance.rs:191-201
    (2, 8, 2, 3, 4, 0),       # :207-221 multi-head
    (2, 8, 2, 0, 2, 0),       # :228-240 partial rotation
    (2, 8, 4, 1, 2, 0),       # :247-260 GQA-shaped head count
    (2, 8, 4, 1, 2, 1),       # half-split
    (32, 256, 64, 0, 4, 0),   # tiny block Q
    (32, 256, 64, 0, 4, 1),
    (5, 4096, 128, 2048, 32, 0),
    (5, 4096, 128, 2048, 32, 1),
    (7, 4096, 64, 100, 32, 0),   # partial: 64 of 128
    (7, 4096, 64, 100, 32, 1),
    (3, 30, 6, 5, 5, 0),      # odd widths: scalar path
    (3, 30, 6, 5, 5, 1),
    (4, 24, 4, 0, 2, 1),      # half = 2: scalar half-split
]


@pytest.mark.parametrize("rows,cols,dim,offset,heads,half_split", ROPE_CASES)
def test_rope_cases(dev, orc, rows, cols, dim, offset, heads, half_split):
    from magnetar_hip import ops
    x = orc.hashed_values(rows * cols, 71).reshape(rows, cols)
    kw = dict(position_offset=offset, half_split=half_split)
    got = ops.rope(dev, dev.upload(x), ops.rope_params(dim, heads, **kw)).numpy()
    p = orc.rope_params(dim, heads, **kw)
    want, st = orc.rope(x, p)
    assert st == 0
    err = rope_pair_err(x, got, want, p)
    print(f"rope {rows}x{cols} dim {dim} heads {heads} split {half_split}: {err:.3e}")
    assert err <= ROPE_TOL


def test_rope_partial_rotary_and_scalings(dev, orc):
    from magnetar_hip import ops
    x = orc.hashed_values(9 * 512, 72).reshape(9, 512)
    cases = [
        dict(rotated_pairs=16),
        dict(banded_factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
             original_context_length=8192.0),
        dict(yarn_factor=4.0, yarn_low=3.0, yarn_high=20.0, amplitude=1.1),
        dict(yarn_factor=4.0, yarn_low=7.0, yarn_high=7.0, amplitude=1.0),
        dict(scale=0.25, base=500000.0),
    ]
    for kw in cases:
        got = ops.rope(dev, dev.upload(x), ops.rope_params(128, 4, position_offset=3000,
                                                           **kw)).numpy()
        p = orc.rope_params(128, 4, position_offset=3000, **kw)
        want, st = orc.rope(x, p)
        assert st == 0
        err = rope_pair_err(x, got, want, p)
        print(f"rope {kw}: {err:.3e}")
        assert err <= ROPE_TOL


def test_rope_rejects_bad_shapes(dev):
    from magnetar_hip import ops, MagnetarHipError
    x = dev.upload(np.zeros((2, 12), np.float32))
    for kw in [dict(dimension=3, head_count=1), dict(dimension=8, head_count=5),
               dict(dimension=8, head_count=3), dict(dimension=0, head_count=1)]:
        with pytest.raises(MagnetarHipError) as err:
            ops.rope(dev, x, ops.rope_params(kw["dimension"], kw["head_count"]))
        assert err.value.code == "ShapeUnsupported"
    with pytest.raises(MagnetarHipError):
        ops.rope(dev, x, ops.rope_params(4, 1, base=-1.0))


def test_rope_baseline_shape(dev, orc):
    """[8192, 32 x 128], theta 10000, positions 0..8191."""
    from magnetar_hip import ops
    x = orc.normal(8192 * 4096, 73).reshape(8192, 4096)
    got = ops.rope(dev, dev.upload(x), ops.rope_params(128, 32)).numpy()
    p = orc.rope_params(128, 32)
    want, st = orc.rope(x, p)
    err = rope_pair_err(x, got, want, p)
    print(f"rope [8192,4096]: max pair-relative err {err:.3e}")
    assert err <= ROPE_TOL


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (8195, 2048), (9000, 1024)])
def test_rmsnorm_many_rows_match_few_rows_bits(dev, orc, rows, cols):
    """Many rows with one shared gain may take a kernel that normalises several
    rows per workgroup; every row must still get the bits a call on that row
    alone produces (same per-row reduction order)."""
    from magnetar_hip import ops
    x = orc.normal(rows * cols, 801 + cols).reshape(rows, cols)
    w = orc.normal(cols, 802, 1.0, 0.1)
    dw = dev.upload(w)
    got = ops.rmsnorm(dev, dev.upload(x), dw, 1e-5).numpy()
    for r0 in (0, 1, rows // 2 + 1, rows - 3):
        part = ops.rmsnorm(dev, dev.upload(np.ascontiguousarray(x[r0:r0 + 3])), dw, 1e-5).numpy()
        assert_bitexact(got[r0:r0 + 3], part)
