"""GPU parity: streaming kernels (add, bias-add, mul, mul-scalar, silu,
silu-mul, scale), the f16/bf16 path and the embedding gather, against the CPU
oracle on identical seeded inputs.

Bars (north star): add/mul/bias-add/scale/embedding/half add-mul bit-exact;
silu and silu-mul within 1e-6 elementwise relative error (they differ from
the oracle only in the last bits of expf).
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact, assert_half_result, is_half_nan, max_rel_err

pytestmark = pytest.mark.gpu

SILU_TOL = 1e-6


def view(dev, base, offset_elems, shape):
    """An unowned DeviceArray `offset_elems` f32 elements into `base`."""
    from magnetar_hip.device import DeviceArray
    return DeviceArray(dev, base.ptr + 4 * offset_elems, shape, np.float32, owned=False)


SIZES = [1, 3, 4, 5, 255, 1000, 4099, 65536 + 7, 1 << 20]


@pytest.mark.parametrize("n", SIZES)
def test_add_mul_bitexact(dev, orc, n):
    from magnetar_hip import ops
    a = orc.hashed_values(n, 1) * 7.0
    b = orc.hashed_values(n, 2) * 3.0
    da, db = dev.upload(a), dev.upload(b)
    for name, fn in (("add", ops.add), ("mul", ops.mul)):
        expected, st = getattr(orc, name)(a, b)
        assert st == 0
        assert_bitexact(fn(dev, da, db).numpy(), expected, f"{name} n={n}")


def test_reference_fixtures(dev, orc):
    """The reference's own add / mul / silu inputs (src/tests_conformance.rs:59-136)."""
    from magnetar_hip import ops
    a = np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(2, 3)
    b = np.array([6, 5, 4, 3, 2, 1], np.float32).reshape(2, 3)
    assert_bitexact(ops.add(dev, dev.upload(a), dev.upload(b)).numpy(), a + b)
    assert_bitexact(ops.mul(dev, dev.upload(a), dev.upload(b)).numpy(), a * b)
    a2 = np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(3, 2)
    bias = np.array([100, 1000], np.float32)
    assert_bitexact(ops.bias_add(dev, dev.upload(a2), dev.upload(bias)).numpy(),
                    np.array([[101, 1002], [103, 1004], [105, 1006]], np.float32))
    x = np.array([-2.0, -0.5, 0.0, 0.5, 1.0, 2.0], np.float32).reshape(2, 3)
    expected, _ = orc.silu(x)
    assert max_rel_err(ops.silu(dev, dev.upload(x)).numpy(), expected, 1e-37) <= SILU_TOL


@pytest.mark.parametrize("n", [5, 1000, 4099])
def test_unaligned_views_take_the_scalar_path(dev, orc, n):
    from magnetar_hip import ops
    a = orc.hashed_values(n, 3)
    b = orc.hashed_values(n, 4)
    base_a, base_b = dev.upload(np.concatenate([[0], a]).astype(np.float32)), \
        dev.upload(np.concatenate([[0], b]).astype(np.float32))
    out = dev.zeros((n + 1,))
    va, vb, vo = view(dev, base_a, 1, (n,)), view(dev, base_b, 1, (n,)), view(dev, out, 1, (n,))
    ops.add(dev, va, vb, out=vo)
    assert_bitexact(vo.numpy(), orc.add(a, b)[0], "unaligned add")
    ops.silu(dev, va, out=vo)
    assert max_rel_err(vo.numpy(), orc.silu(a)[0], 1e-37) <= SILU_TOL


@pytest.mark.parametrize("rows,cols", [(3, 2), (7, 5), (64, 4096), (33, 1028), (1, 11008)])
def test_bias_add_bitexact(dev, orc, rows, cols):
    from magnetar_hip import ops
    a = orc.hashed_values(rows * cols, 5).reshape(rows, cols)
    bias = orc.hashed_values(cols, 6)
    expected, st = orc.bias_add(a, bias)
    assert st == 0
    assert_bitexact(ops.bias_add(dev, dev.upload(a), dev.upload(bias)).numpy(), expected)


def test_bias_add_rejects_non_dividing_cols(dev):
    from magnetar_hip import ops, MagnetarHipError
    a = dev.upload(np.zeros(10, np.float32))
    bias = dev.upload(np.zeros(3, np.float32))
    with pytest.raises(MagnetarHipError) as err:
        ops.bias_add(dev, a, bias)
    assert err.value.code == "ShapeUnsupported"


@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_mul_scalar_and_scale_bitexact(dev, orc, n):
    from magnetar_hip import ops
    a = orc.hashed_values(n, 7) * 11.0
    s = np.array([0.3712], np.float32)
    assert_bitexact(ops.mul_scalar(dev, dev.upload(a), dev.upload(s)).numpy(),
                    orc.mul_scalar(a, s)[0])
    assert_bitexact(ops.scale(dev, dev.upload(a), 64.0).numpy(), orc.scale(a, 64.0)[0])


@pytest.mark.parametrize("n", SIZES)
def test_silu_and_silu_mul(dev, orc, n):
    from magnetar_hip import ops
    x = orc.normal(n, 8, 0.0, 4.0)
    up = orc.hashed_values(n, 9)
    assert max_rel_err(ops.silu(dev, dev.upload(x)).numpy(), orc.silu(x)[0], 1e-37) <= SILU_TOL
    got = ops.silu_mul(dev, dev.upload(x), dev.upload(up)).numpy()
    assert max_rel_err(got, orc.silu_mul(x, up)[0], 1e-37) <= SILU_TOL


def test_silu_special_values(dev, orc):
    from magnetar_hip import ops
    x = np.array([0.0, -0.0, 1e-30, -1e-30, 100.0, -100.0, 89.0, -89.0, 1e30, -1e30,
                  np.inf, -np.inf, np.nan], np.float32)
    got = ops.silu(dev, dev.upload(x)).numpy()
    want = orc.silu(x)[0]
    finite = np.isfinite(want)
    assert max_rel_err(got[finite], want[finite], 1e-37) <= SILU_TOL
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.signbit(got[finite]), np.signbit(want[finite]))


def test_elementwise_at_baseline_size(dev, orc):
    """[8192, 4096] (the BASELINE shape): add, mul, bias and residual add
    bit-exact, silu and silu-mul within the tolerance, against the oracle."""
    from magnetar_hip import ops
    shape = (8192, 4096)
    n = shape[0] * shape[1]
    a = orc.normal(n, 71, 0.0, 1.0).reshape(shape)
    b = orc.normal(n, 72, 0.0, 1.0).reshape(shape)
    bias = orc.normal(shape[1], 73, 0.0, 1.0)
    da, db = dev.upload(a), dev.upload(b)
    assert_bitexact(ops.add(dev, da, db).numpy(), orc.add(a, b)[0], "add")
    assert_bitexact(ops.mul(dev, da, db).numpy(), orc.mul(a, b)[0], "mul")
    assert_bitexact(ops.bias_add(dev, da, dev.upload(bias)).numpy(), orc.bias_add(a, bias)[0], "bias")
    assert max_rel_err(ops.silu(dev, da).numpy(), orc.silu(a)[0], 1e-37) <= SILU_TOL
    assert max_rel_err(ops.silu_mul(dev, da, db).numpy(), orc.silu_mul(a, b)[0], 1e-37) <= SILU_TOL


def test_embedding_table_past_2_gib(dev, orc):
    """The C3 lookup: 8192 ids into a [128000, 4096] table (2.1 GB, so row
    offsets pass 2^31 bytes), bit-exact. Entry (r, c) holds the bit pattern
    r * 4096 + c (distinct, finite, denormal for r < 2048)."""
    from magnetar_hip import ops
    vocab, dim = 128000, 4096
    table = (np.arange(vocab, dtype=np.uint32)[:, None] * dim
             + np.arange(dim, dtype=np.uint32)[None, :]).view(np.float32)
    ids = orc.token_ids(8192, 74, vocab)
    ids[:3] = [vocab - 1, 0, 2048]
    got = ops.embedding(dev, dev.upload(table), dev.upload(ids)).numpy()
    assert dev.check_flags() == 0
    want, st = orc.embedding(table, ids)
    assert st == 0
    assert_bitexact(got, want)


# ---- half precision ---------------------------------------------------------

HALF = {"f16": 0, "bf16": 1}


def test_half_reference_fixtures(dev, orc):
    """src/tests_conformance.rs:2349-2423: the reference's inputs, its exact model."""
    from magnetar_hip import ops
    a = np.array([1.0, 2.5, 3.0, -4.25, 0.1, 100.0], np.float32)
    b = np.array([6.0, 0.2, 4.0, 3.0, 0.2, -99.5], np.float32)
    for dname, dt in HALF.items():
        ha, hb = orc.encode_half(a, dt), orc.encode_half(b, dt)
        for op in ("add", "mul"):
            got = ops.half_binary(dev, dev.upload(ha), dev.upload(hb), op, dt).numpy()
            assert_bitexact(got, orc.half_binary(ha, hb, dt, op), f"{op}-{dname}")


@pytest.mark.parametrize("dname", ["f16", "bf16"])
@pytest.mark.parametrize("op", ["add", "mul"])
def test_half_random_bit_patterns(dev, orc, dname, op):
    """Uniformly random 16-bit patterns (subnormals, infinities and NaNs
    included), bit for bit: NaN results too (a NaN operand's payload,
    quieted; the negative default NaN from inf - inf or 0 * inf), except that
    NaN op NaN may keep either operand's quieted payload, which is all the
    reference's arithmetic fixes there."""
    dt = HALF[dname]
    rng = np.random.default_rng(11 + dt)
    n = (1 << 22) + 5
    ha = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    hb = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    got = ops_half(dev, ha, hb, op, dt)
    want = orc.half_binary(ha, hb, dt, op)
    nan_w = is_half_nan(want, dt)
    assert nan_w.sum() > 1000  # NaN payloads are exercised
    both = assert_half_result(orc, got, want, ha, hb, dt, f"{op}-{dname}")
    assert both > 30  # NaN op NaN is exercised (bf16: ~64 of 4M pairs)
    # This build's convention on top of the admissible set: the first operand's.
    assert_bitexact(got, want, f"{op}-{dname} (first-operand convention)")


def ops_half(dev, ha, hb, op, dt):
    from magnetar_hip import ops
    return ops.half_binary(dev, dev.upload(ha), dev.upload(hb), op, dt).numpy()


@pytest.mark.parametrize("dname", ["f16", "bf16"])
def test_half_all_pairs_of_one_operand(dev, orc, dname):
    """Every 16-bit pattern against a fixed set of partners: covers each
    exponent's rounding, overflow and gradual underflow."""
    dt = HALF[dname]
    all_bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    partners = orc.encode_half(np.array([1.0, -1.0, 0.5, 3.0, 1e-3, 65504.0, 1e-7, 0.0,
                                         -0.0, 2.0 ** -14, 1.0009765625], np.float32), dt)
    for p in partners:
        hb = np.full(all_bits.shape, p, np.uint16)
        for op in ("add", "mul"):
            got = ops_half(dev, all_bits, hb, op, dt)
            want = orc.half_binary(all_bits, hb, dt, op)
            assert_bitexact(got, want, f"{op}-{dname} partner={p:#x}")


@pytest.mark.parametrize("dname", ["f16", "bf16"])
def test_half_codec_on_device(dev, orc, dname):
    """Device encode/decode against the reference codec: all 65536 decodes, and
    encodes of every f32 sign/exponent with rounding-critical mantissas."""
    from magnetar_hip import ops
    dt = HALF[dname]
    all_bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    dec = ops.decode_half(dev, dev.upload(all_bits), dt).numpy()
    assert_bitexact(dec, orc.decode_half(all_bits, dt), f"decode-{dname}")
    sign_exp = (np.arange(512, dtype=np.uint32) << 23)
    hi = np.arange(1 << 10, dtype=np.uint32) << 13
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF, 0x7FFF, 0x8000, 0x8001, 0xFFFF],
                    np.uint32)
    mant = (hi[:, None] | lows[None, :]).reshape(-1) & 0x7FFFFF
    f32_bits = (sign_exp[:, None] | mant[None, :]).reshape(-1)
    x = f32_bits.view(np.float32)
    enc = ops.encode_half(dev, dev.upload(x), dt).numpy()
    assert_bitexact(enc, orc.encode_half(x, dt), f"encode-{dname}")


def test_half_at_baseline_size(dev, orc):
    """64M-element f16 and bf16 add/mul (the BASELINE shape) against the oracle."""
    n = 1 << 26
    x = orc.normal(n, 21)
    y = orc.normal(n, 22)
    for dname, dt in HALF.items():
        ha, hb = orc.encode_half(x, dt), orc.encode_half(y, dt)
        for op in ("add", "mul"):
            assert_bitexact(ops_half(dev, ha, hb, op, dt), orc.half_binary(ha, hb, dt, op),
                            f"{op}-{dname} 64M")


# ---- embedding ----------------------------------------------------------------

def test_embedding_reference_fixture(dev, orc):
    """src/tests_conformance.rs:138-161."""
    from magnetar_hip import ops
    table = np.array([0.0, 0.1, 0.2, 1.0, 1.1, 1.2, 2.0, 2.1, 2.2, 3.0, 3.1, 3.2],
                     np.float32).reshape(4, 3)
    ids = np.array([0.0, 2.0, 1.0], np.float32)
    got = ops.embedding(dev, dev.upload(table), dev.upload(ids)).numpy()
    assert dev.check_flags() == 0
    assert_bitexact(got, table[[0, 2, 1]])


@pytest.mark.parametrize("vocab,dim,num", [(1024, 256, 32), (128, 4096, 100), (50, 7, 9),
                                           (32000, 4096, 1), (1000, 1028, 33), (64, 2048, 300)])
def test_embedding_bitexact(dev, orc, vocab, dim, num):
    from magnetar_hip import ops
    table = orc.normal(vocab * dim, 31).reshape(vocab, dim)
    ids = orc.token_ids(num, 32, vocab)
    got = ops.embedding(dev, dev.upload(table), dev.upload(ids)).numpy()
    assert dev.check_flags() == 0
    want, st = orc.embedding(table, ids)
    assert st == 0
    assert_bitexact(got, want)


@pytest.mark.parametrize("bad", [5.0, 4.0, -1.0, 1.5, float("nan"), float("inf"), 1e30])
def test_embedding_invalid_id_fails(dev, orc, bad):
    """src/tests_conformance.rs:163-175: an out-of-range id fails the lookup."""
    from magnetar_hip import ops, MagnetarHipError
    table = np.zeros((4, 8), np.float32)
    ids = np.array([0.0, bad], np.float32)
    assert orc.embedding(table, ids)[1] == 1
    ops.embedding(dev, dev.upload(table), dev.upload(ids))
    with pytest.raises(MagnetarHipError) as err:
        dev.check_flags()
    assert err.value.code == "ShapeUnsupported"
    assert "not a valid in-range non-negative integer" in err.value.detail
    assert dev.check_flags() == 0  # the check clears the flag


def test_embedding_negative_zero_is_row_zero(dev, orc):
    from magnetar_hip import ops
    table = orc.normal(4 * 8, 33).reshape(4, 8)
    ids = np.array([-0.0, 3.0], np.float32)
    got = ops.embedding(dev, dev.upload(table), dev.upload(ids)).numpy()
    assert dev.check_flags() == 0
    assert_bitexact(got, orc.embedding(table, ids)[0])
