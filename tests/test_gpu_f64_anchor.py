"""GPU: per-kernel elementwise error anchored on f64.

For each kernel at its BASELINE shape, the device's result and the CPU
oracle's (the reference's f32 order: k ascending, sequential sums) are both
measured against an f64 evaluation of the same mathematics on the same f32
inputs (tests/f64_reference.py). The measure is the elementwise relative error
over the entries with |exact| >= 1e-3 * max |exact| (an entry that cancels to
~0 has no meaningful relative error). The bar, asserted per kernel:

    device-vs-f64  <=  max(1e-4, ORACLE_FACTOR * oracle-vs-f64)

i.e. the device is within the north star's 1e-4 of the exact result, or no
further from it than f32 arithmetic in the reference's own order gets (with a
factor for the spread of a maximum over many entries: two f32 summation orders
of the same sum have errors of the same distribution, not the same maximum).
Matmul is also held to the order-independent forward-error bound
|C - C^| <= gamma_k (|A||B|) entry by entry (Higham eq. 3.5), which no
summation order may exceed. Each test prints both figures.
"""
import numpy as np
import pytest

import f64_reference as x64
from conftest import max_normwise_err

pytestmark = pytest.mark.gpu

ORACLE_FACTOR = 2.0
BAR = 1e-4


def check(name, gpu_err, orc_err):
    bound = max(BAR, ORACLE_FACTOR * orc_err)
    print(f"[f64] {name}: device {gpu_err:.2e}, oracle {orc_err:.2e}, bound {bound:.2e}", flush=True)
    assert gpu_err <= bound, (name, gpu_err, orc_err)


@pytest.mark.parametrize("size,rows", [(1024, 1024), (2048, 64), (4096, 24), (8192, 12)])
def test_matmul_square(dev, orc, size, rows):
    """BASELINE config 2's square products (A, B ~U(-1,1)): the whole product
    at 1024, evenly spaced sampled rows beyond."""
    from magnetar_hip import ops
    from reference_chain import matmul as oracle_matmul
    a = orc.uniform(size * size, 21, -1.0, 1.0).reshape(size, size)
    b = orc.uniform(size * size, 22, -1.0, 1.0).reshape(size, size)
    got = ops.matmul(dev, dev.upload(a), dev.upload(b)).numpy()
    idx = np.linspace(0, size - 1, rows).astype(int)
    exact = x64.matmul(a[idx], b)
    if rows == size:
        orc_rows = oracle_matmul(orc, a, b)
    else:
        orc_rows = np.concatenate([orc.matmul_rows(a, b, int(r), int(r) + 1) for r in idx])
    check(f"matmul {size}^3", x64.rel_err_significant(got[idx], exact),
          x64.rel_err_significant(orc_rows, exact))
    bound = x64.gamma(size) * x64.abs_product(a[idx], b)
    assert np.all(np.abs(got[idx] - exact) <= bound), "gamma_k bound"


def test_matmul_skinny(dev, orc):
    """1 x 4096 x 11008 (the decode GEMV, split-k with an ordered reduction)."""
    from magnetar_hip import ops
    a = orc.uniform(4096, 11, -1.0, 1.0).reshape(1, 4096)
    b = orc.uniform(4096 * 11008, 12, -1.0, 1.0).reshape(4096, 11008)
    got = ops.matmul(dev, dev.upload(a), dev.upload(b)).numpy()
    exact = x64.matmul(a, b)
    want, _ = orc.matmul(a, b)
    check("matmul 1x4096x11008", x64.rel_err_significant(got, exact),
          x64.rel_err_significant(want, exact))
    assert np.all(np.abs(got - exact) <= x64.gamma(4096) * x64.abs_product(a, b))


def test_rmsnorm_and_softmax_c3(dev, orc):
    """C3: [8192, 4096] rmsnorm (eps 1e-5, gain ~N(1, 0.1)) and softmax of
    ~N(0, 4) rows."""
    from magnetar_hip import ops
    x = orc.normal(8192 * 4096, 31).reshape(8192, 4096)
    w = orc.normal(4096, 32, 1.0, 0.1)
    got = ops.rmsnorm(dev, dev.upload(x), dev.upload(w), 1e-5).numpy()
    want, _ = orc.rmsnorm(x, w, 1e-5)
    exact = x64.rmsnorm(x, w, 1e-5)
    check("rmsnorm [8192,4096]", x64.rel_err_significant(got, exact),
          x64.rel_err_significant(want, exact))
    del got, want, exact
    s = orc.normal(8192 * 4096, 33, 0.0, 2.0).reshape(8192, 4096)
    got = ops.softmax_rows(dev, dev.upload(s)).numpy()
    dev.check_flags()
    want, _ = orc.softmax_rows(s)
    exact = x64.softmax_rows(s)
    check("softmax [8192,4096]", x64.rel_err_significant(got, exact),
          x64.rel_err_significant(want, exact))


def test_rope_c3(dev, orc):
    """C3: [8192, 32 x 128] at positions 0..8191 (theta 10000, interleaved)."""
    from magnetar_hip import ops
    x = orc.normal(8192 * 4096, 34).reshape(8192, 4096)
    p = orc.rope_params(128, 32)
    got = ops.rope(dev, dev.upload(x), ops.rope_params(128, 32)).numpy()
    want, _ = orc.rope(x, p)
    exact = x64.rope(orc, x, p)
    check("rope [8192,4096]", x64.rel_err_significant(got, exact),
          x64.rel_err_significant(want, exact))


def test_attention_c4_prefill(dev, orc):
    """C4: B4 H32 d128 S2048 causal; one head of each batch element (the heads
    the C4 parity test checks)."""
    from magnetar_hip import ops
    from reference_chain import attention as oracle_attention
    B, S, H, d = 4, 2048, 32, 128
    q = orc.normal(B * S * H * d, 41).reshape(B * S, H * d)
    k = orc.normal(B * S * H * d, 42).reshape(B * S, H * d)
    v = orc.normal(B * S * H * d, 43).reshape(B * S, H * d)
    p = ops.attention_params(S, S, H, d, causal=True, batch=B)
    got = ops.attention(dev, dev.upload(q), dev.upload(k), dev.upload(v), p).numpy()
    worst_gpu = worst_orc = 0.0
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        h0 = b * 7 % H
        cols = slice(h0 * d, (h0 + 1) * d)
        qs, ks, vs = q[rows], k[rows], v[rows]
        exact = x64.attention(qs, ks, vs, S, H, H, d, heads=(h0, h0 + 1))[:, cols]
        op = orc.attention_params(S, S, H, d, causal=True)
        want, st = orc.attention(qs, ks, vs, op, heads=(h0, h0 + 1))
        assert st == 0
        worst_gpu = max(worst_gpu, x64.rel_err_significant(got[rows, cols], exact))
        worst_orc = max(worst_orc, x64.rel_err_significant(want[:, cols], exact))
    check("attention C4 prefill", worst_gpu, worst_orc)


def test_attention_c4_decode(dev, orc):
    """C4 decode: one query against 4096 keys, batch 8, every head."""
    from magnetar_hip import ops
    B, KV, H, d = 8, 4096, 32, 128
    q = orc.normal(B * H * d, 51).reshape(B, H * d)
    k = orc.normal(B * KV * H * d, 52).reshape(B * KV, H * d)
    v = orc.normal(B * KV * H * d, 53).reshape(B * KV, H * d)
    p = ops.attention_params(1, KV, H, d, causal=True, batch=B)
    got = ops.attention(dev, dev.upload(q), dev.upload(k), dev.upload(v), p).numpy()
    exact = np.concatenate([x64.attention(q[b:b + 1], k[b * KV:(b + 1) * KV], v[b * KV:(b + 1) * KV],
                                          1, H, H, d) for b in range(B)])
    from reference_chain import attention as oracle_attention
    want = np.concatenate([oracle_attention(orc, q[b:b + 1], k[b * KV:(b + 1) * KV],
                                            v[b * KV:(b + 1) * KV],
                                            orc.attention_params(1, KV, H, d, causal=True))
                           for b in range(B)])
    check("attention C4 decode", x64.rel_err_significant(got, exact),
          x64.rel_err_significant(want, exact))


def _block_case(dev, orc, s, seed, seq, position, cache_rows, history_seed=None):
    from magnetar_hip.decoder import DecoderBlock
    from reference_chain import reference_block
    from test_gpu_decoder import weights_for
    w = weights_for(orc, s, seed)
    block = DecoderBlock(dev, s, w, cache_rows=cache_rows, max_seq=seq)
    kv = s.kv_heads * s.head_dim
    kc = np.zeros((cache_rows, kv), np.float32)
    vc = np.zeros((cache_rows, kv), np.float32)
    if history_seed is not None and position:
        kc[:position] = orc.normal(position * kv, history_seed, 0.0, 0.5).reshape(position, kv)
        vc[:position] = orc.normal(position * kv, history_seed + 1, 0.0, 0.5).reshape(position, kv)
        block.k_cache = dev.upload(kc)
        block.v_cache = dev.upload(vc)
    ids = orc.token_ids(seq, seed + 1, s.vocab)
    got = block.forward(dev.upload(ids), position).numpy()
    dev.check_flags()
    want, _, _ = reference_block(orc, s, w, ids, position, kc, vc)
    exact, _, _ = x64.block(orc, s, w, ids, position, kc, vc)
    assert max_normwise_err(got, want) <= 1e-4
    return x64.rel_err_significant(got, exact), x64.rel_err_significant(want, exact)


def test_block_c1(dev, orc):
    """C1: the tiny block, seq 32 at position 0."""
    from magnetar_hip.decoder import Shapes
    s = Shapes(vocab=1024, hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=688)
    check("block C1 seq 32", *_block_case(dev, orc, s, 100, 32, 0, 64))


def test_block_c5_decode(dev, orc):
    """C5 decode: one token at position 2048 against 2048 cached rows."""
    from magnetar_hip.decoder import Shapes
    s = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    check("block C5 decode @2048", *_block_case(dev, orc, s, 300, 1, 2048, 2049, history_seed=301))


def test_block_c5_prefill(dev, orc):
    """C5 prefill: 512 tokens at position 0."""
    from magnetar_hip.decoder import Shapes
    s = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    check("block C5 prefill 512", *_block_case(dev, orc, s, 400, 512, 0, 512))
