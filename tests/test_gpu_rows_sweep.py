"""GPU parity: seeded random shapes for RMSNorm, softmax and RoPE against the
CPU oracle (RMSNorm and softmax within 1e-4 max relative error, RoPE within
1e-6 of each rotated pair's norm, pass-through columns unchanged)."""
import numpy as np
import pytest

from conftest import max_rel_err, sweep_seeds
from test_gpu_rows import rope_pair_err

pytestmark = pytest.mark.gpu


def _cols(rng):
    # widths across the one-wave, four-wave and looped kernels, aligned or not
    return int(rng.choice([int(rng.integers(1, 64)), 4 * int(rng.integers(1, 300)),
                           4 * int(rng.integers(1000, 4200)), int(rng.integers(1, 20000))]))


@pytest.mark.parametrize("seed", sweep_seeds(30))
def test_rmsnorm_random(dev, orc, seed):
    from magnetar_hip import ops
    rng = np.random.default_rng(20_000 + seed)
    rows, cols = int(rng.integers(1, 300)), _cols(rng)
    mode = seed % 3  # no gain, one gain row, a gain per row
    x = orc.normal(rows * cols, 7000 + seed).reshape(rows, cols)
    w = None if mode == 0 else orc.normal(cols if mode == 1 else rows * cols, 7100 + seed, 1.0, 0.1)
    stride = cols if mode == 2 else 0
    eps = float(rng.choice([1e-6, 1e-5, 1e-3]))
    got = ops.rmsnorm(dev, dev.upload(x), dev.upload(w) if w is not None else None, eps,
                      weight_row_stride=stride).numpy()
    want, st = orc.rmsnorm(x, w, eps, weight_row_stride=stride)
    assert st == 0
    err = max_rel_err(got, want)
    print(f"seed {seed}: rmsnorm [{rows},{cols}] mode {mode}: {err:.2e}")
    assert err <= 1e-4


@pytest.mark.parametrize("seed", sweep_seeds(30))
def test_softmax_random(dev, orc, seed):
    from magnetar_hip import ops
    rng = np.random.default_rng(30_000 + seed)
    rows, cols = int(rng.integers(1, 300)), _cols(rng)
    x = orc.normal(rows * cols, 8000 + seed, 0.0, float(rng.choice([0.5, 2.0, 8.0]))).reshape(rows, cols)
    got = ops.softmax_rows(dev, dev.upload(x)).numpy()
    assert dev.check_flags() == 0
    want, st = orc.softmax_rows(x)
    assert st == 0
    err = max_rel_err(got, want)
    print(f"seed {seed}: softmax [{rows},{cols}]: {err:.2e}")
    assert err <= 1e-4


@pytest.mark.parametrize("seed", sweep_seeds(30))
def test_rope_random(dev, orc, seed):
    from magnetar_hip import ops
    rng = np.random.default_rng(40_000 + seed)
    heads = int(rng.choice([1, 2, 3, 4, 8, 32]))
    hw = 2 * int(rng.integers(1, 80))
    dim = 2 * int(rng.integers(1, hw // 2 + 1))
    rows = int(rng.integers(1, 200))
    kw = dict(position_offset=int(rng.integers(0, 9000)), half_split=int(rng.integers(0, 2)),
              base=float(rng.choice([10000.0, 500000.0, 1e6])),
              scale=float(rng.choice([1.0, 1.0, 0.5, 0.125])))
    x = orc.normal(rows * heads * hw, 9000 + seed).reshape(rows, heads * hw)
    got = ops.rope(dev, dev.upload(x), ops.rope_params(dim, heads, **kw)).numpy()
    p = orc.rope_params(dim, heads, **kw)
    want, st = orc.rope(x, p)
    assert st == 0
    err = rope_pair_err(x, got, want, p)
    print(f"seed {seed}: rope rows {rows} heads {heads} width {hw} dim {dim} {kw}: {err:.2e}")
    assert err <= 1e-6
