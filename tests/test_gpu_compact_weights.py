"""GPU: compact bf16 weights (`execute-native-half-precision`, reference
src/kernels.rs:1665-1723, src/executor.rs:384-399, :1323-1364) and on-device
greedy selection (src/kernels.rs:4437-4488, src/kernels.cu:1808-1866).

Bars: a product, lookup or block over a compact weight is bit-identical to the
f32 path over the widened weight (the widening is exact and the arithmetic is
the f32 path's); greedy selection is an index, exact against the oracle.
"""
import numpy as np
import pytest

from conftest import max_normwise_err

pytestmark = pytest.mark.gpu


def bf16_values(rng, shape, scale=1.0):
    """Random f32 values that are exact bf16 values, and their bit patterns."""
    v = (rng.standard_normal(shape) * scale).astype(np.float32)
    bits = (v.view(np.uint32) >> 16).astype(np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32), bits


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("m,k,n,ta,tb,mode", [
    (1, 4096, 4096, False, False, 0),    # decode GEMV
    (3, 1000, 516, False, False, 2),     # GEMV, ragged k, residual
    (8, 256, 64, False, False, 1),       # GEMV, bias
    (4, 2048, 2056, False, False, 1),    # GEMV, 8 columns per lane, bias
    (2, 512, 1032, False, False, 2),     # GEMV, 8 columns per lane, one split, residual
    (32, 256, 688, False, False, 2),     # row-blocked GEMV, residual
    (9, 300, 130, False, False, 0),      # MFMA, ragged edges
    (64, 2048, 256, False, False, 0),    # MFMA with split-k
    (512, 512, 512, False, False, 2),
    (400, 2050, 1900, False, False, 2),  # MFMA stream-K
    (40, 96, 72, False, True, 1),        # b stored [n, k]
    (33, 64, 47, True, True, 0),
    (1, 64, 10, False, False, 0),        # n % 4 != 0: tile path
])
def test_compact_matmul_equals_the_f32_path(dev, m, k, n, ta, tb, mode):
    from magnetar_hip import ops
    rng = np.random.default_rng(m * 1000 + n)
    a = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    wv, wb = bf16_values(rng, (n, k) if tb else (k, n), 0.05)
    addend = None
    if mode == 1:
        addend = dev.upload(rng.standard_normal(n).astype(np.float32))
    elif mode == 2:
        addend = dev.upload(rng.standard_normal((m, n)).astype(np.float32))
    da = dev.upload(a)
    want = ops.matmul(dev, da, dev.upload(wv), ta, tb, addend, mode).numpy()
    got = ops.matmul_bf16w(dev, da, dev.upload(wb), ta, tb, addend, mode).numpy()
    assert same_bits(got, want)


def test_compact_matmul_against_the_oracle(dev, orc):
    from magnetar_hip import ops
    rng = np.random.default_rng(5)
    a = rng.standard_normal((17, 333)).astype(np.float32)
    wv, wb = bf16_values(rng, (333, 200), 0.1)
    got = ops.matmul_bf16w(dev, dev.upload(a), dev.upload(wb)).numpy()
    want, st = orc.matmul(a, wv)
    assert st == 0
    assert max_normwise_err(got, want) <= 1e-4


@pytest.mark.parametrize("vocab,dim", [(1000, 4096), (64, 256), (50, 6)])
def test_compact_embedding_equals_the_f32_lookup(dev, orc, vocab, dim):
    import magnetar_hip
    from magnetar_hip import ops
    rng = np.random.default_rng(vocab + dim)
    tv, tb = bf16_values(rng, (vocab, dim))
    ids = dev.upload(orc.token_ids(37, 9, vocab))
    want = ops.embedding(dev, dev.upload(tv), ids).numpy()
    got = ops.embedding_bf16w(dev, dev.upload(tb), ids).numpy()
    dev.check_flags()
    assert same_bits(got, want)
    ops.embedding_bf16w(dev, dev.upload(tb), dev.upload(np.array([float(vocab)], np.float32)))
    with pytest.raises(magnetar_hip.MagnetarHipError):
        dev.check_flags()


@pytest.mark.parametrize("seq,position", [(1, 30), (4, 10), (40, 0)])
def test_compact_decoder_block_equals_the_f32_block(dev, orc, seq, position):
    """The block over bf16 weights equals the block over their f32 widening,
    bit for bit: decode GEMV sets, the fused embedding + rmsnorm and prefill
    tiles all read the compact matrices."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    s = Shapes(vocab=700, hidden=512, heads=8, kv_heads=2, head_dim=64, ffn=1376)
    rng = np.random.default_rng(seq)
    w = {}
    for name, shape in s.weight_shapes().items():
        if name.endswith("norm"):
            w[name] = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
        else:
            w[name] = bf16_values(rng, shape, 0.02)[0]
    kc = orc.normal(64 * 128, 11, 0.0, 0.5).reshape(64, 128)
    vc = orc.normal(64 * 128, 12, 0.0, 0.5).reshape(64, 128)
    ids = dev.upload(orc.token_ids(seq, 13, 700))
    outs = []
    for compact in (False, True):
        block = DecoderBlock(dev, s, w, cache_rows=64, max_seq=40, bf16_weights=compact)
        block.k_cache, block.v_cache = dev.upload(kc), dev.upload(vc)
        outs.append((block.forward(ids, position).numpy(), block.k_cache.numpy(),
                     block.v_cache.numpy()))
    dev.check_flags()
    for f32_part, bf16_part in zip(*outs):
        assert same_bits(bf16_part, f32_part)


# ---- the executor's compact weights ----

@pytest.fixture(scope="module")
def provider():
    import magnetar_hip
    p = magnetar_hip.Provider()
    yield p
    p.close()


def inv(kernel, inputs, output, attrs=None):
    from magnetar_hip import KernelInvocation, TensorRef
    return KernelInvocation(kernel, [TensorRef(i) for i in inputs], [TensorRef(output)], attrs or {})


def test_write_weight_tensor_stores_exact_bf16_matrices_compact(provider):
    ex = provider.execution_api()
    rng = np.random.default_rng(1)
    wv, _ = bf16_values(rng, (256, 512), 0.05)            # 131072 exact values
    assert ex.write_weight_tensor("cw.w", wv)
    assert not ex.write_weight_tensor("cw.small", wv[:64])   # < 65536 values
    inexact = wv.copy()
    inexact[3, 3] += np.float32(1e-6)
    assert not ex.write_weight_tensor("cw.inexact", inexact)
    assert not ex.write_weight_tensor("cw.vector", wv.ravel())   # not a matrix
    assert same_bits(ex.read_tensor("cw.w"), wv)
    assert same_bits(ex.read_tensor_rows("cw.w", 10, 3), wv[10:13])
    assert ex.resident_shape("cw.w") == ((256, 512), 0)

    a = rng.standard_normal((3, 256)).astype(np.float32)
    ex.write_tensor("cw.a", a)
    ex.write_tensor("cw.wf", wv)
    for kernel, extra in (("matmul", {}), ("matmul-residual", {})):
        ins = ["cw.a", "cw.w"] + (["cw.res"] if kernel == "matmul-residual" else [])
        ins_f = ["cw.a", "cw.wf"] + (["cw.res"] if kernel == "matmul-residual" else [])
        ex.write_tensor("cw.res", np.ones((3, 512), np.float32))
        ex.execute(inv(kernel, ins, "cw.y"))
        ex.execute(inv(kernel, ins_f, "cw.yf"))
        assert same_bits(ex.read_tensor("cw.y"), ex.read_tensor("cw.yf")), kernel
    ex.execute(inv("gated-matmul", ["cw.a", "cw.w", "cw.w"], "cw.g"))
    ex.execute(inv("gated-matmul", ["cw.a", "cw.wf", "cw.wf"], "cw.gf"))
    assert same_bits(ex.read_tensor("cw.g"), ex.read_tensor("cw.gf"))

    # An embedding table reads compact; ids are any f32 tensor.
    ex.write_tensor("cw.ids", np.array([0.0, 255.0, 7.0], np.float32))
    ex.execute(inv("embedding", ["cw.w", "cw.ids"], "cw.e"))
    assert same_bits(ex.read_tensor("cw.e"), wv[[0, 255, 7]])

    # Any other use stores the weight as f32 first, for good.
    ex.write_tensor("cw.z", np.zeros((256, 512), np.float32))
    ex.execute(inv("add", ["cw.w", "cw.z"], "cw.sum"))
    assert same_bits(ex.read_tensor("cw.sum"), wv)
    assert same_bits(ex.read_tensor("cw.w"), wv)
    ex.execute(inv("matmul", ["cw.a", "cw.w"], "cw.y2"))
    ex.execute(inv("matmul", ["cw.a", "cw.wf"], "cw.y2f"))
    assert same_bits(ex.read_tensor("cw.y2"), ex.read_tensor("cw.y2f"))


# ---- greedy selection ----

@pytest.mark.parametrize("cols", [1, 7, 1000, 32000, 128256])
def test_greedy_select_matches_the_oracle(dev, orc, cols):
    from magnetar_hip import ops
    rng = np.random.default_rng(cols)
    rows = 3
    logits = rng.standard_normal((rows, cols)).astype(np.float32)
    logits[1, rng.integers(0, cols, max(1, cols // 100))] = np.nan
    logits[2, rng.integers(0, cols, max(1, cols // 100))] = np.inf
    logits[0, rng.integers(0, cols, 3)] = logits[0].max()        # ties
    d = dev.upload(logits)
    cases = [((), 0.0), ((), 0.7), ((), -1.5), (((0, cols // 2),), 0.0),
             (((0, 1), (cols // 3, cols // 3 + 5), (cols - 1, cols)), 2.0)]
    for row in range(rows):
        for excluded, t in cases:
            want = orc.greedy_select(logits[row], excluded, t)
            got = ops.greedy_select(dev, d, row, excluded, t)
            assert got == want, (row, excluded, t)


def test_greedy_select_edge_cases(dev):
    import magnetar_hip
    from magnetar_hip import ops
    nan, inf = np.nan, np.inf
    d = dev.upload(np.array([[nan, inf, -inf, nan], [-0.0, 0.0, -1.0, -0.0]], np.float32))
    assert ops.greedy_select(dev, d, 0) is None
    assert ops.greedy_select(dev, d, 1) == 0
    assert ops.greedy_select(dev, d, 1, excluded=[(0, 4)]) is None
    with pytest.raises(magnetar_hip.MagnetarHipError):
        ops.greedy_select(dev, d, 2)


def test_select_greedy_column_through_the_executor(provider, orc):
    ex = provider.execution_api()
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((2, 32000)).astype(np.float32)
    ex.write_tensor("gs.logits", logits)
    for row in range(2):
        assert ex.select_greedy_column("gs.logits", row) == int(np.argmax(logits[row]))
        top = int(np.argmax(logits[row]))
        assert ex.select_greedy_column("gs.logits", row, [(top, top + 1)]) == \
            orc.greedy_select(logits[row], [(top, top + 1)])
    assert ex.select_greedy_column("gs.logits", 5) is None
    assert ex.select_greedy_column("gs.missing", 0) is None
