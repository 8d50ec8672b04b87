"""GPU parity: f32 matmul (MFMA tiles and the decode GEMV) against the CPU oracle.

Bar (north star): within 1e-4 max relative error, measured normwise:
max |gpu - cpu| / max |cpu| over the output (an output entry near zero after
cancellation has no meaningful elementwise relative error; the normwise
measure still catches a dropped or doubled k term, ~|a||b| / max|C| ~ 1e-3 at
these sizes). Fused bias / residual epilogues must be bit-identical to the
unfused matmul followed by add (src/tests_conformance.rs:293-408).
"""
import numpy as np
import pytest

from conftest import assert_bitexact, max_normwise_err, max_rel_err_significant

pytestmark = pytest.mark.gpu

TOL = 1e-4


def run(dev, a, b, ta=False, tb=False, addend=None, mode=0):
    from magnetar_hip import ops
    return ops.matmul(dev, dev.upload(a), dev.upload(b), ta, tb,
                      dev.upload(addend) if addend is not None else None, mode).numpy()


def test_reference_fixtures(dev, orc):
    """src/tests_conformance.rs:262-288 (plain and transposed a)."""
    a = np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(2, 3)
    b = np.array([1, 0, 0, 1, 1, 1], np.float32).reshape(3, 2)
    assert_bitexact(run(dev, a, b), orc.matmul(a, b)[0])
    at = np.array([1, 4, 2, 5, 3, 6], np.float32).reshape(3, 2)
    assert_bitexact(run(dev, at, b, ta=True), orc.matmul(at, b, True)[0])


@pytest.mark.parametrize("m,k,n,ta", [(1, 1000, 70, False), (1, 37, 33, False),
                                      (3, 129, 65, False), (5, 64, 1, False),
                                      (4, 50, 40, True)])
def test_reference_uneven_shapes(dev, orc, m, k, n, ta):
    """src/tests_conformance.rs:447-481, with its `values` generator."""
    a = orc.values(m * k, 1).reshape((k, m) if ta else (m, k))
    b = orc.values(k * n, 2).reshape(k, n)
    err = max_normwise_err(run(dev, a, b, ta), orc.matmul(a, b, ta)[0])
    assert err <= TOL


SHAPES = [(128, 128, 128), (256, 512, 384), (130, 33, 70), (129, 257, 131), (64, 4096, 64),
          (9, 100, 300), (300, 7, 5), (512, 1024, 768), (1000, 1000, 1000), (32, 256, 688)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_mfma_shapes_and_transposes(dev, orc, m, k, n, ta, tb):
    a = orc.uniform(m * k, 100 + m, -1.0, 1.0).reshape((k, m) if ta else (m, k))
    b = orc.uniform(k * n, 200 + n, -1.0, 1.0).reshape((n, k) if tb else (k, n))
    want, st = orc.matmul(a, b, ta, tb)
    assert st == 0
    err = max_normwise_err(run(dev, a, b, ta, tb), want)
    print(f"matmul {m}x{k}x{n} ta={ta} tb={tb}: normwise err {err:.2e}")
    assert err <= TOL


def test_integer_inputs_are_exact(dev, orc):
    """Small-integer operands: every partial sum is an exactly representable
    integer, so any summation order gives the exact product."""
    rng = np.random.default_rng(5)
    a = rng.integers(-8, 9, (200, 300)).astype(np.float32)
    b = rng.integers(-8, 9, (300, 150)).astype(np.float32)
    exact = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    assert_bitexact(run(dev, a, b), exact)
    a1 = a[:3]
    assert_bitexact(run(dev, a1, b[:, :148]), exact[:3, :148])


@pytest.mark.parametrize("m,k,n", [(1, 4096, 256), (130, 64, 96), (1, 300, 40), (8, 128, 64)])
def test_fused_addend_is_bit_identical_to_unfused(dev, orc, m, k, n):
    from magnetar_hip import ops
    a = dev.upload(orc.values(m * k, 3).reshape(m, k))
    b = dev.upload(orc.values(k * n, 4).reshape(k, n))
    bias = dev.upload(orc.values(n, 5))
    resid = dev.upload(orc.values(m * n, 6).reshape(m, n))
    plain = ops.matmul(dev, a, b)
    unfused_bias = ops.bias_add(dev, plain, bias).numpy()
    unfused_res = ops.add(dev, plain, resid).numpy()
    assert_bitexact(ops.matmul(dev, a, b, addend=bias, addend_mode=1).numpy(), unfused_bias)
    assert_bitexact(ops.matmul(dev, a, b, addend=resid, addend_mode=2).numpy(), unfused_res)


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
def test_decode_gemv_rows(dev, orc, m):
    k, n = 4096, 1024
    a = orc.uniform(m * k, 7, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 8, -1.0, 1.0).reshape(k, n)
    err = max_normwise_err(run(dev, a, b), orc.matmul(a, b)[0])
    assert err <= TOL


def test_skinny_decode_baseline_shape(dev, orc):
    """M=1, K=4096, N=11008."""
    a = orc.uniform(4096, 11, -1.0, 1.0).reshape(1, 4096)
    b = orc.uniform(4096 * 11008, 12, -1.0, 1.0).reshape(4096, 11008)
    err = max_normwise_err(run(dev, a, b), orc.matmul(a, b)[0])
    print(f"matmul 1x4096x11008: normwise err {err:.2e}")
    assert err <= TOL


def test_zero_inner_dimension(dev, orc):
    a = np.zeros((3, 0), np.float32)
    b = np.zeros((0, 4), np.float32)
    from magnetar_hip import ops
    bias = np.arange(4, dtype=np.float32)
    got = ops.matmul(dev, dev.upload(a), dev.upload(b), addend=dev.upload(bias),
                     addend_mode=1).numpy()
    assert_bitexact(got, np.tile(bias, (3, 1)))


SQUARE_TILES = {1024: (64, 64), 2048: (128, 128), 4096: (256, 256), 8192: (256, 256)}


@pytest.mark.parametrize("size", [1024, 2048, 4096, 8192])
def test_square_baseline_sizes(dev, orc, size):
    """BASELINE config 2's square products. 1024^3 against the whole oracle
    product (rows split over host threads, values unchanged); the larger ones
    at 16 sampled rows against the oracle exactly as it sums them, plus a
    checksum of the whole product, C x = A (B x), in f64. The elementwise
    relative error over entries of at least 1e-3 of the largest is printed
    beside the normwise bar."""
    from magnetar_hip import ops
    from reference_chain import matmul as oracle_matmul
    from magnetar_hip import ops as _ops
    plan = _ops.matmul_plan(dev, size, size, size)
    assert plan["path"] == "tiles" and plan["tile"] == SQUARE_TILES[size], plan
    assert plan["splits"] == 1 and not plan["stream_k"], plan
    a = orc.uniform(size * size, 21, -1.0, 1.0).reshape(size, size)
    b = orc.uniform(size * size, 22, -1.0, 1.0).reshape(size, size)
    c = ops.matmul(dev, dev.upload(a), dev.upload(b)).numpy()
    if size <= 1024:
        want = oracle_matmul(orc, a, b)
        err = max_normwise_err(c, want)
        print(f"matmul {size}^3 whole product: normwise {err:.2e}, "
              f"elementwise (|ref| >= 1e-3 max) {max_rel_err_significant(c, want):.2e}")
        assert err <= TOL
    rows = np.linspace(0, size - 1, 16).astype(int)
    worst = 0.0
    for r in rows:
        want = orc.matmul_rows(a, b, int(r), int(r) + 1)
        err = max_normwise_err(c[r:r + 1], want)
        worst = max(worst, err)
        assert err <= TOL
    x = np.random.default_rng(0).standard_normal(size)
    lhs = c.astype(np.float64) @ x
    rhs = a.astype(np.float64) @ (b.astype(np.float64) @ x)
    err = np.max(np.abs(lhs - rhs)) / np.max(np.abs(rhs))
    print(f"matmul {size}^3 sampled rows {worst:.2e}, checksum err {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("m,k,n,mode", [(4000, 64, 4064, 0), (4000, 96, 4064, 1), (4064, 40, 4000, 2)])
def test_large_tile_path_ragged_edges_and_addends(dev, orc, m, k, n, mode):
    """Products of about one 256 x 256 tile per CU take the 8-wave 256-tile
    kernel (asserted); ragged edges and both addend forms against the oracle,
    and the fused addend bit-identical to matmul + add."""
    from magnetar_hip import ops
    plan = ops.matmul_plan(dev, m, k, n)
    assert plan["tile"] == (256, 256) and plan["splits"] == 1 and not plan["stream_k"], plan
    a = orc.uniform(m * k, 31 + m, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 32 + n, -1.0, 1.0).reshape(k, n)
    addend = None
    if mode == 1:
        addend = orc.uniform(n, 33, -1.0, 1.0)
    elif mode == 2:
        addend = orc.uniform(m * n, 34, -1.0, 1.0).reshape(m, n)
    da, db = dev.upload(a), dev.upload(b)
    dadd = dev.upload(addend) if addend is not None else None
    got = ops.matmul(dev, da, db, addend=dadd, addend_mode=mode).numpy()
    want, st = orc.matmul(a, b, addend=addend, addend_mode=mode)
    assert st == 0
    assert max_normwise_err(got, want) <= 1e-4
    if mode:
        plain = ops.matmul(dev, da, db)
        summed = (ops.add(dev, plain, dadd) if mode == 2 else ops.bias_add(dev, plain, dadd)).numpy()
        assert np.array_equal(got.view(np.uint32), summed.view(np.uint32))


@pytest.mark.parametrize("m,k,n,mode", [(16, 1028, 256, 0), (24, 1100, 256, 1), (32, 258, 688, 2),
                                        (32, 102, 300, 0), (16, 4096, 1024, 2)])
def test_row_blocked_gemv(dev, orc, m, k, n, mode):
    """Small products of 16-32 rows with k > 1024 or k % 4 != 0 run as blocks
    of 8 rows on the split-k GEMV: against the oracle, and each block of 8
    rows bit-identical to the 8-row GEMV of those rows alone (same slicing of
    k, same summation order)."""
    from magnetar_hip import ops
    assert ops.matmul_plan(dev, m, k, n)["path"] == "gemv_row_blocks"
    assert ops.matmul_plan(dev, 8, k, n)["path"] == "gemv"
    a = orc.uniform(m * k, 41 + m, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 42 + n, -1.0, 1.0).reshape(k, n)
    addend = None
    if mode == 1:
        addend = orc.uniform(n, 43, -1.0, 1.0)
    elif mode == 2:
        addend = orc.uniform(m * n, 44, -1.0, 1.0).reshape(m, n)
    db = dev.upload(b)
    got = ops.matmul(dev, dev.upload(a), db, addend=dev.upload(addend) if addend is not None else None,
                     addend_mode=mode).numpy()
    want, st = orc.matmul(a, b, addend=addend, addend_mode=mode)
    assert st == 0
    assert max_normwise_err(got, want) <= TOL
    for r in range(0, m, 8):
        part = None
        if mode == 1:
            part = dev.upload(addend)
        elif mode == 2:
            part = dev.upload(np.ascontiguousarray(addend[r:r + 8]))
        block = ops.matmul(dev, dev.upload(np.ascontiguousarray(a[r:r + 8])), db, addend=part,
                           addend_mode=mode).numpy()
        assert_bitexact(got[r:r + 8], block)


@pytest.mark.parametrize("m,k,n,mode", [(16, 256, 256, 0), (24, 688, 256, 1), (32, 256, 688, 2),
                                        (32, 100, 300, 0), (32, 1024, 2048, 2), (16, 4, 36, 1),
                                        (24, 1024, 4, 0)])
def test_small_mfma_tiles(dev, orc, m, k, n, mode):
    """Small products of 16-32 rows with k <= 1024 (k % 4 == 0) run in one
    launch of 32 x 32 MFMA tiles, k split over the workgroup's 16 waves:
    against the oracle (both addend forms), ragged column tiles and short
    last k ranges included, and every 16-row block bit-identical to the
    product of those rows alone (an output's sum depends only on its own row
    and column)."""
    from magnetar_hip import ops
    plan = ops.matmul_plan(dev, m, k, n)
    assert plan["path"] == "small_tiles" and plan["tile"] == (32, 32) and plan["waves"] == 16, plan
    a = orc.uniform(m * k, 45 + m, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 46 + n, -1.0, 1.0).reshape(k, n)
    addend = None
    if mode == 1:
        addend = orc.uniform(n, 47, -1.0, 1.0)
    elif mode == 2:
        addend = orc.uniform(m * n, 48, -1.0, 1.0).reshape(m, n)
    db = dev.upload(b)
    got = ops.matmul(dev, dev.upload(a), db, addend=dev.upload(addend) if addend is not None else None,
                     addend_mode=mode).numpy()
    want, st = orc.matmul(a, b, addend=addend, addend_mode=mode)
    assert st == 0
    err = max_normwise_err(got, want)
    print(f"small tiles [{m},{k},{n}] mode {mode}: normwise err {err:.2e}")
    assert err <= TOL
    for r in range(0, m - 15, 8):
        part = None
        if mode == 1:
            part = dev.upload(addend)
        elif mode == 2:
            part = dev.upload(np.ascontiguousarray(addend[r:r + 16]))
        block = ops.matmul(dev, dev.upload(np.ascontiguousarray(a[r:r + 16])), db, addend=part,
                           addend_mode=mode).numpy()
        assert_bitexact(got[r:r + 16], block)


@pytest.mark.parametrize("m,k,n,mode,tile,stream", [
    (200, 2050, 1900, 0, 128, True), (200, 2050, 1900, 1, 128, True), (201, 2050, 1901, 2, 128, True),
    (200, 4096, 2500, 1, 128, True), (130, 512, 3000, 2, 64, True),
    (400, 1024, 1900, 2, 128, False), (130, 512, 1900, 1, 64, False), (40, 4096, 4096, 1, 64, False)])
def test_stream_k_products(dev, orc, m, k, n, mode, tile, stream):
    """Products whose tiles cannot fill the device split k: stream-K (equal
    runs of (tile, k slice) units per workgroup, partial tiles summed in k
    order) or whole k splits, on the 64-, and 128-tile kernels (the plan is
    asserted; the 256-tile stream-K is the prefill projection below): ragged
    edges, a short last run, against the oracle, deterministic, and the fused
    addend bit-identical to matmul + add."""
    from magnetar_hip import ops
    plan = ops.matmul_plan(dev, m, k, n)
    assert plan["tile"] == (tile, tile) and plan["stream_k"] == stream, plan
    assert stream or plan["splits"] > 1, plan
    a = orc.uniform(m * k, 51 + m, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 52 + n, -1.0, 1.0).reshape(k, n)
    addend = None
    if mode == 1:
        addend = orc.uniform(n, 53, -1.0, 1.0)
    elif mode == 2:
        addend = orc.uniform(m * n, 54, -1.0, 1.0).reshape(m, n)
    da, db = dev.upload(a), dev.upload(b)
    dadd = dev.upload(addend) if addend is not None else None
    got = ops.matmul(dev, da, db, addend=dadd, addend_mode=mode).numpy()
    want, st = orc.matmul(a, b, addend=addend, addend_mode=mode)
    assert st == 0
    err = max_normwise_err(got, want)
    print(f"stream-K {m}x{k}x{n} mode {mode}: normwise err {err:.2e}")
    assert err <= TOL
    again = ops.matmul(dev, da, db, addend=dadd, addend_mode=mode).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))  # deterministic
    if mode:
        plain = ops.matmul(dev, da, db)
        summed = (ops.add(dev, plain, dadd) if mode == 2 else ops.bias_add(dev, plain, dadd)).numpy()
        assert np.array_equal(got.view(np.uint32), summed.view(np.uint32))


def test_stream_k_prefill_projection(dev, orc):
    """The gate/up projection of a 512-token Llama-2-7B prefill (512 x 4096
    x 11008, 86 tiles of 256 x 256, stream-K): 16 sampled rows against the
    oracle and a checksum of the whole product, C x = A (B x), in f64."""
    from magnetar_hip import ops
    m, k, n = 512, 4096, 11008
    plan = ops.matmul_plan(dev, m, k, n)
    assert plan["tile"] == (256, 256) and plan["stream_k"], plan
    a = orc.uniform(m * k, 61, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 62, -1.0, 1.0).reshape(k, n)
    c = ops.matmul(dev, dev.upload(a), dev.upload(b)).numpy()
    for r in np.linspace(0, m - 1, 16).astype(int):
        assert max_normwise_err(c[r:r + 1], orc.matmul_rows(a, b, int(r), int(r) + 1)) <= TOL
    x = np.random.default_rng(1).standard_normal(n)
    lhs = c.astype(np.float64) @ x
    rhs = a.astype(np.float64) @ (b.astype(np.float64) @ x)
    assert np.max(np.abs(lhs - rhs)) / np.max(np.abs(rhs)) <= TOL


@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
def test_large_tile_path_with_transposed_operands(dev, orc, ta, tb):
    """The 256 x 256 tile kernel with A stored [k, m] and/or B stored [n, k]:
    ragged edges, against the oracle, and bit-identical to the same product
    with the operands stored untransposed (same tiles, same k order)."""
    from magnetar_hip import ops
    m, k, n = 4000, 96, 4064
    assert ops.matmul_plan(dev, m, k, n, ta, tb)["tile"] == (256, 256)
    a = orc.uniform(m * k, 91, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 92, -1.0, 1.0).reshape(k, n)
    a_in = np.ascontiguousarray(a.T) if ta else a
    b_in = np.ascontiguousarray(b.T) if tb else b
    got = ops.matmul(dev, dev.upload(a_in), dev.upload(b_in), ta, tb).numpy()
    want, st = orc.matmul(a, b)
    assert st == 0
    assert max_normwise_err(got, want) <= TOL
    plain = ops.matmul(dev, dev.upload(a), dev.upload(b)).numpy()
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))


@pytest.mark.parametrize("m,k,n,waves,splits", [(2000, 1056, 3000, 8, 2), (3200, 512, 3968, 4, 1)])
@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
def test_128_tiles_one_slice_per_barrier_with_transposed_operands(dev, orc, m, k, n, waves, splits, ta, tb):
    """The 128 x 128 tiles in launches of more workgroups than CUs, one slice
    per barrier, every wave issuing part of the next slice's direct loads: the
    8-wave tiles with a k split (ragged edges, slices of 544 and 512 k) and the
    4-wave tiles two to a CU. Stored transposed, the operands give the bits of
    the untransposed product, whose sampled rows match the oracle."""
    from magnetar_hip import ops
    plan = ops.matmul_plan(dev, m, k, n, ta, tb)
    assert plan["tile"] == (128, 128) and plan["waves"] == waves and plan["splits"] == splits, plan
    assert not plan["stream_k"], plan
    a = orc.uniform(m * k, 93, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 94, -1.0, 1.0).reshape(k, n)
    a_in = np.ascontiguousarray(a.T) if ta else a
    b_in = np.ascontiguousarray(b.T) if tb else b
    got = ops.matmul(dev, dev.upload(a_in), dev.upload(b_in), ta, tb).numpy()
    plain = ops.matmul(dev, dev.upload(a), dev.upload(b)).numpy()
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))
    for r in np.linspace(0, m - 1, 8).astype(int):
        assert max_normwise_err(plain[r:r + 1], orc.matmul_rows(a, b, int(r), int(r) + 1)) <= TOL


@pytest.mark.parametrize("m,k,n", [(1024, 1024, 1024), (1024, 1056, 1024), (1000, 1000, 1000)])
@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
def test_64_tiles_with_transposed_operands(dev, orc, m, k, n, ta, tb):
    """The 64 x 64 tiles in two k groups, whose split of each slice's groups
    of 8 k is uneven on every fourth slice: the untransposed product takes
    whole four-slice steps (a partial last step at k = 1056, edge tiles at
    1000), the transposed ones slice by slice; every path follows the same
    split, so the bits match. Sampled rows against the oracle."""
    from magnetar_hip import ops
    assert ops.matmul_plan(dev, m, k, n, ta, tb)["tile"] == (64, 64)
    a = orc.uniform(m * k, 95, -1.0, 1.0).reshape(m, k)
    b = orc.uniform(k * n, 96, -1.0, 1.0).reshape(k, n)
    a_in = np.ascontiguousarray(a.T) if ta else a
    b_in = np.ascontiguousarray(b.T) if tb else b
    got = ops.matmul(dev, dev.upload(a_in), dev.upload(b_in), ta, tb).numpy()
    plain = ops.matmul(dev, dev.upload(a), dev.upload(b)).numpy()
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))
    for r in np.linspace(0, m - 1, 8).astype(int):
        assert max_normwise_err(plain[r:r + 1], orc.matmul_rows(a, b, int(r), int(r) + 1)) <= TOL


def _offset_view(dev, host):
    """`host` on the device 4 bytes past a 16-byte boundary (and the owner to keep alive)."""
    from magnetar_hip.device import DeviceArray
    owner = dev.upload(np.concatenate([np.zeros(1, np.float32), host.ravel()]))
    return DeviceArray(dev, owner.ptr + 4, host.shape, np.float32, owned=False), owner


@pytest.mark.parametrize("m,k,n,ta,tb", [(512, 256, 512, False, False), (512, 256, 512, True, True),
                                         (256, 160, 384, False, True), (96, 200, 160, False, False)])
def test_unaligned_operands_give_the_aligned_bits(dev, orc, m, k, n, ta, tb):
    """Misaligned operands take the register-staged slices (bounds-checked
    scalar loads), aligned ones the direct global-to-LDS slices; both sum k
    in the same order, so the products are bit-identical."""
    from magnetar_hip import ops
    a = orc.normal(m * k, 301).reshape((k, m) if ta else (m, k))
    b = orc.normal(k * n, 302).reshape((n, k) if tb else (k, n))
    aligned = ops.matmul(dev, dev.upload(a), dev.upload(b), ta, tb).numpy()
    av, a_owner = _offset_view(dev, a)
    bv, b_owner = _offset_view(dev, b)
    shifted = ops.matmul(dev, av, bv, ta, tb).numpy()
    assert_bitexact(shifted, aligned)
    ref, _ = orc.matmul(a, b, ta, tb)
    assert max_normwise_err(aligned, ref) < TOL
