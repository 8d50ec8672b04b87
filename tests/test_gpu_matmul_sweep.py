"""GPU parity: seeded random matmul shapes against the CPU oracle.

Each case draws a shape (tiny, around tile edges, or mid-size), transposes and
an addend mode from its own seed, so a failure names a reproducible case. The
bars: within 1e-4 normwise of the oracle; for MFMA-sized products the
transposed storage gives the same bits; compact bf16 weights give the bits
of the f32 path over the widened weights.
"""
import numpy as np
import pytest

from conftest import assert_bitexact, max_normwise_err, sweep_seeds

pytestmark = pytest.mark.gpu

EDGES_M = [127, 128, 129, 255, 256, 257, 383, 384, 511, 512, 513]
EDGES_N = [127, 128, 129, 255, 256, 257, 384, 512, 640]
EDGES_K = [1, 31, 32, 33, 63, 64, 96, 100, 257, 512]


def draw(seed):
    rng = np.random.default_rng(seed)
    kind = seed % 3
    if kind == 0:
        m, k, n = (int(v) for v in rng.integers(1, 70, 3))
    elif kind == 1:
        m, n, k = int(rng.choice(EDGES_M)), int(rng.choice(EDGES_N)), int(rng.choice(EDGES_K))
    else:
        m, k, n = (int(v) for v in rng.integers(33, 700, 3))
    return m, k, n, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), int(rng.integers(0, 3))


@pytest.mark.parametrize("seed", sweep_seeds(60))
def test_random_shape(dev, orc, seed):
    from magnetar_hip import ops
    m, k, n, ta, tb, mode = draw(seed)
    a = orc.normal(m * k, 1000 + seed).reshape((k, m) if ta else (m, k))
    b = orc.normal(k * n, 2000 + seed).reshape((n, k) if tb else (k, n))
    add = None
    if mode == 1:
        add = orc.normal(n, 3000 + seed)
    elif mode == 2:
        add = orc.normal(m * n, 3000 + seed).reshape(m, n)
    dadd = dev.upload(add) if add is not None else None
    got = ops.matmul(dev, dev.upload(a), dev.upload(b), ta, tb, dadd, mode).numpy()
    want, st = orc.matmul(a, b, ta, tb, add, mode)
    assert st == 0
    err = max_normwise_err(got, want)
    print(f"seed {seed}: [{m},{k},{n}] ta={ta} tb={tb} mode={mode} err {err:.2e}")
    assert err < 1e-4
    if m > 32:
        flipped = ops.matmul(dev, dev.upload(np.ascontiguousarray(a.T)),
                             dev.upload(np.ascontiguousarray(b.T)), not ta, not tb, dadd,
                             mode).numpy()
        assert_bitexact(flipped, got)
    if n % 4 == 0:
        bits16 = (b.view(np.uint32) >> 16).astype(np.uint16)
        widened = (bits16.astype(np.uint32) << 16).view(np.float32)
        f32 = ops.matmul(dev, dev.upload(a), dev.upload(widened), ta, tb, dadd, mode).numpy()
        compact = ops.matmul_bf16w(dev, dev.upload(a), dev.upload(bits16), ta, tb, dadd, mode).numpy()
        assert_bitexact(compact, f32)
