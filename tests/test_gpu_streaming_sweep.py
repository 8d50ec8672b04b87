"""GPU parity: seeded random lengths and misaligned views for the streaming
ops, bit-exact against the CPU oracle (f32 add/mul/bias-add/mul-scalar,
f16/bf16 add/mul) or within 1e-6 (silu, silu-mul). Random lengths exercise
the ragged tails; a 4-byte (f32) or 2-byte (half) offset the unaligned paths.
"""
import numpy as np
import pytest

from conftest import assert_bitexact, max_rel_err, sweep_seeds

pytestmark = pytest.mark.gpu


def _view(dev, host, shift, half=None):
    """`host` on the device, `shift` elements past an aligned start, and its owner."""
    from magnetar_hip.device import DeviceArray
    pad = np.zeros(shift, host.dtype)
    owner = dev.upload(np.concatenate([pad, host.ravel()]), half=half)
    view = DeviceArray(dev, owner.ptr + shift * host.dtype.itemsize, host.shape, host.dtype,
                       half=half, owned=False)
    return view, owner


def _draw(seed):
    rng = np.random.default_rng(50_000 + seed)
    n = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 5000)),
                        int(rng.integers(5000, 300_000))]))
    return n, int(rng.integers(0, 2)), rng


@pytest.mark.parametrize("seed", sweep_seeds(24))
def test_f32_streaming_random(dev, orc, seed):
    from magnetar_hip import ops
    n, shift, rng = _draw(seed)
    a = orc.normal(n, 100 + seed)
    b = orc.normal(n, 200 + seed)
    da, oa = _view(dev, a, shift)
    db, ob = _view(dev, b, shift)
    assert_bitexact(ops.add(dev, da, db).numpy(), orc.add(a, b)[0])
    assert_bitexact(ops.mul(dev, da, db).numpy(), orc.mul(a, b)[0])
    s = orc.normal(1, 300 + seed)
    assert_bitexact(ops.mul_scalar(dev, da, dev.upload(s)).numpy(), orc.mul_scalar(a, s)[0])
    assert max_rel_err(ops.silu(dev, da).numpy(), orc.silu(a)[0], 1e-37) <= 1e-6
    assert max_rel_err(ops.silu_mul(dev, da, db).numpy(), orc.silu_mul(a, b)[0], 1e-37) <= 1e-6
    cols = int(rng.integers(1, 300))
    rows = max(1, n // cols)
    m = orc.normal(rows * cols, 400 + seed).reshape(rows, cols)
    bias = orc.normal(cols, 500 + seed)
    dm, om = _view(dev, m, shift)
    assert_bitexact(ops.bias_add(dev, dm, dev.upload(bias)).numpy(), orc.bias_add(m, bias)[0])


@pytest.mark.parametrize("seed", sweep_seeds(24))
def test_half_streaming_random(dev, orc, seed):
    from magnetar_hip import ops, MHIP_F16, MHIP_BF16
    n, shift, _ = _draw(seed)
    dtype = MHIP_F16 if seed % 2 == 0 else MHIP_BF16
    a = orc.encode_half(orc.normal(n, 600 + seed, 0.0, 3.0), dtype)
    b = orc.encode_half(orc.normal(n, 700 + seed, 0.0, 3.0), dtype)
    da, oa = _view(dev, a, shift, dtype)
    db, ob = _view(dev, b, shift, dtype)
    for op in ("add", "mul"):
        got = ops.half_binary(dev, da, db, op, dtype).numpy()
        assert_bitexact(got, orc.half_binary(a, b, dtype, op))
