"""GPU: the in-place KV cache append (`kv-write`, reference src/kernels.rs:2270-2325,
src/executor.rs:1366-1420) and attention bounded by `key_count` over a store
whose tail is NaN (src/tests_conformance.rs:1068-1139).

Bars: kv-write is a copy, bit-exact; attention 1e-4 normwise against the oracle
over exactly the history rows.
"""
import numpy as np
import pytest

from conftest import max_normwise_err

pytestmark = pytest.mark.gpu


def test_kv_write_writes_rows_in_place_and_rejects_overruns(dev):
    import magnetar_hip
    from magnetar_hip import ops
    store = dev.upload(np.zeros((4, 2), np.float32))
    rows = dev.upload(np.array([[1, 2], [3, 4]], np.float32))
    ops.kv_write(dev, store, rows, 1)
    assert store.numpy().ravel().tolist() == [0, 0, 1, 2, 3, 4, 0, 0]
    with pytest.raises(magnetar_hip.MagnetarHipError) as err:
        ops.kv_write(dev, store, rows, 3)
    assert err.value.code == "ShapeUnsupported"
    assert "exceeds the store's 4 rows" in str(err.value)
    assert store.numpy().ravel().tolist() == [0, 0, 1, 2, 3, 4, 0, 0]


def test_kv_write_unaligned_rows_bitexact(dev, orc):
    """Odd widths take the scalar path; any f32 bit pattern is copied as is."""
    from magnetar_hip import ops
    rng = np.random.default_rng(7)
    store_h = rng.standard_normal((37, 5)).astype(np.float32)
    rows_h = rng.integers(0, 2**32, (9, 5), dtype=np.uint64).astype(np.uint32).view(np.float32)
    store = dev.upload(store_h)
    ops.kv_write(dev, store, dev.upload(rows_h), 20)
    want = store_h.copy()
    want[20:29] = rows_h
    assert np.array_equal(store.numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("case,history,heads,kv_heads,dim,capacity", [
    (0, 300, 14, 2, 64, 307),      # grouped decode, seven query heads per KV head
    (1, 12500, 2, 1, 4, 12507),    # a long history of narrow heads
    # Stores large enough for the decode's double-length key chunks (chosen
    # from the capacity when the key count is bounded), one and two query
    # heads per KV head.
    (2, 3000, 32, 32, 128, 8200),
    (3, 5000, 32, 16, 128, 16400),
])
def test_key_count_attention_ignores_the_store_tail(dev, orc, case, history, heads, kv_heads, dim,
                                                    capacity):
    from magnetar_hip import ops
    width = kv_heads * dim
    q = orc.attention_values(heads * dim, 10 * case + 1).reshape(1, heads * dim)
    k = orc.attention_values(history * width, 10 * case + 2).reshape(history, width)
    v = orc.attention_values(history * width, 10 * case + 3).reshape(history, width)
    want, st = orc.attention(q, k, v, orc.attention_params(1, history, heads, dim,
                                                           kv_head_count=kv_heads, causal=True))
    assert st == 0

    def with_tail(t):
        out = np.full((capacity, width), np.nan, np.float32)
        out[:history] = t
        return out

    p = ops.attention_params(1, capacity, heads, dim, kv_head_count=kv_heads, causal=True,
                             key_count=history)
    got = ops.attention(dev, dev.upload(q), dev.upload(with_tail(k)), dev.upload(with_tail(v)), p)
    got = got.numpy()
    assert np.all(np.isfinite(got))
    assert max_normwise_err(got, want) <= 1e-4


def test_decode_steps_append_with_kv_write(dev, orc):
    """A decode loop that appends each step's K/V rows with kv-write and attends
    with key_count = position + 1 matches attention over the full history."""
    from magnetar_hip import ops
    heads, dim, steps, capacity = 4, 64, 6, 16
    width = heads * dim
    k_all = orc.normal(steps * width, 11).reshape(steps, width)
    v_all = orc.normal(steps * width, 12).reshape(steps, width)
    kc = dev.upload(np.full((capacity, width), np.nan, np.float32))
    vc = dev.upload(np.full((capacity, width), np.nan, np.float32))
    for t in range(steps):
        ops.kv_write(dev, kc, dev.upload(k_all[t:t + 1]), t)
        ops.kv_write(dev, vc, dev.upload(v_all[t:t + 1]), t)
        q = orc.normal(width, 100 + t).reshape(1, width)
        p = ops.attention_params(1, capacity, heads, dim, causal=True, key_count=t + 1)
        got = ops.attention(dev, dev.upload(q), kc, vc, p).numpy()
        want, _ = orc.attention(q, k_all[:t + 1], v_all[:t + 1],
                                orc.attention_params(1, t + 1, heads, dim, causal=True))
        assert max_normwise_err(got, want) <= 1e-4
