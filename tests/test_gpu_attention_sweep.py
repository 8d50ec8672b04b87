"""GPU parity: seeded random attention shapes against the CPU oracle.

Each case draws the query and key counts, heads, grouping, head size
(MFMA prefill sizes 64 and 128 and others), causal or not, a window, a key
count and a scale from its own seed; within 1e-4 normwise of the oracle.
"""
import numpy as np
import pytest

from conftest import max_normwise_err, sweep_seeds

pytestmark = pytest.mark.gpu


def draw(seed):
    rng = np.random.default_rng(10_000 + seed)
    d = int(rng.choice([64, 128, 64, 128, 32, 96, 16]))
    hkv = int(rng.choice([1, 2, 4]))
    h = hkv * int(rng.choice([1, 2, 4]))
    kv = int(rng.integers(1, 700))
    seq = 1 if seed % 4 == 0 else int(rng.integers(1, kv + 1))
    causal = bool(rng.integers(0, 2))
    window = int(rng.integers(1, 300)) if causal and rng.integers(0, 3) == 0 else None
    key_count = int(rng.integers(seq, kv + 1)) if rng.integers(0, 3) == 0 else None
    scale = float(rng.uniform(0.01, 0.3)) if rng.integers(0, 4) == 0 else None
    return seq, kv, h, hkv, d, causal, window, key_count, scale


@pytest.mark.parametrize("seed", sweep_seeds(48))
def test_random_shape(dev, orc, seed):
    from magnetar_hip import ops
    seq, kv, h, hkv, d, causal, window, key_count, scale = draw(seed)
    q = orc.normal(seq * h * d, 4000 + seed).reshape(seq, h * d)
    k = orc.normal(kv * hkv * d, 5000 + seed).reshape(kv, hkv * d)
    v = orc.normal(kv * hkv * d, 6000 + seed).reshape(kv, hkv * d)
    kw = dict(seq_len=seq, kv_rows=kv, head_count=h, head_dimension=d, kv_head_count=hkv,
              causal=causal, window_size=window, key_count=key_count, scale=scale)
    got = ops.attention(dev, dev.upload(q), dev.upload(k), dev.upload(v),
                        ops.attention_params(**kw)).numpy()
    want, st = orc.attention(q, k, v, orc.attention_params(**kw))
    assert st == 0
    err = max_normwise_err(got, want)
    print(f"seed {seed}: {kw} err {err:.2e}")
    assert err <= 1e-4
