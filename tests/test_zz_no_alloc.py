"""GPU: the allocation-free matmul, mhip_matmul_f32_noalloc, called through the
C ABI. It has no counterpart in the reference; it is mhip_matmul_f32 with the
partial sums in a fixed device array instead of the context's workspace.

Each path that uses scratch (decode GEMV split-k, row-blocked GEMV, 128- and
256-tile split-k, stream-K) is called twice in a row, the second call with a
smaller input (the array keeps the first call's contents), and every output
must equal mhip_matmul_f32's on the same inputs bit for bit, and the oracle's
sampled rows within the matmul bar (1e-4 normwise). A fresh context captures a
split-k product through it (capture refuses the workspace growth the ordinary
entry point needs there), and a product whose partial sums exceed the array is
refused with a clear error.
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact, max_normwise_err

pytestmark = pytest.mark.gpu

TOL = 1e-4
SHAPE_UNSUPPORTED = 1


def _p(arr):
    return ctypes.c_void_p(arr.ptr if arr is not None else 0)


def noalloc(dev, a, b, m, k, n, ta=0, tb=0, addend=None, mode=0, out=None):
    """(status, out) of one mhip_matmul_f32_noalloc call."""
    from magnetar_hip import _lib
    out = out if out is not None else dev.empty((m, n))
    st = _lib.lib().mhip_matmul_f32_noalloc(dev.ctx, _p(a), _p(b), _p(out), m, k, n, ta, tb,
                                            _p(addend), mode)
    return st, out


def operands(dev, orc, m, k, n, ta, tb, mode, seed):
    a = orc.uniform(m * k, seed, -1.0, 1.0).reshape((k, m) if ta else (m, k))
    b = orc.uniform(k * n, seed + 1, -1.0, 1.0).reshape((n, k) if tb else (k, n))
    addend = None
    if mode == 1:
        addend = orc.uniform(n, seed + 2, -1.0, 1.0)
    elif mode == 2:
        addend = orc.uniform(m * n, seed + 2, -1.0, 1.0).reshape(m, n)
    return a, b, addend


# (m, k, n, transpose_a, transpose_b, addend mode) for each path with scratch.
# Each is checked against mhip_matmul_plan_f32 (test_paths_use_the_scratch),
# so a change of the time model cannot move a case off the path it is for.
GEMV = (1, 4096, 11008, 0, 0, 0)          # split-k GEMV
GEMV_ROWS = (5, 4096, 1024, 0, 0, 2)      # split-k GEMV, 5 rows
GEMV_BLOCKS = (16, 1100, 512, 0, 0, 1)    # row blocks of 8 (k > 1024: not the small tiles)
SPLIT_A = (40, 4096, 4096, 0, 0, 0)       # tiles with whole-k splits
SPLIT_B = (400, 1024, 1900, 0, 0, 2)      # tiles with whole-k splits
STREAM_K = (512, 4096, 11008, 0, 0, 0)    # stream-K
TRANSPOSED = (300, 1536, 200, 1, 1, 1)
NO_SPLIT = (1024, 1024, 1024, 0, 0, 0)    # 64-tiles, no scratch: the array is not used

PAIRS = [(STREAM_K, SPLIT_A), (SPLIT_A, SPLIT_B), (SPLIT_B, GEMV), (GEMV, GEMV_ROWS),
         (GEMV_ROWS, GEMV_BLOCKS), (STREAM_K, TRANSPOSED), (SPLIT_A, NO_SPLIT)]


def uses_scratch(plan):
    if plan["path"] in ("gemv", "gemv_row_blocks"):
        return plan["splits"] > 1
    return plan["path"] == "tiles" and (plan["splits"] > 1 or plan["stream_k"])


def test_paths_use_the_scratch(dev):
    """Every case above but NO_SPLIT really goes through the scratch array, on
    the path it is named for."""
    from magnetar_hip import ops
    plan = lambda c: ops.matmul_plan(dev, c[0], c[1], c[2], bool(c[3]), bool(c[4]))
    assert plan(GEMV)["path"] == "gemv" and plan(GEMV)["splits"] > 1, plan(GEMV)
    assert plan(GEMV_ROWS)["path"] == "gemv" and plan(GEMV_ROWS)["splits"] > 1, plan(GEMV_ROWS)
    assert plan(GEMV_BLOCKS)["path"] == "gemv_row_blocks", plan(GEMV_BLOCKS)
    assert plan(GEMV_BLOCKS)["splits"] > 1, plan(GEMV_BLOCKS)
    for case in (SPLIT_A, SPLIT_B):
        p = plan(case)
        assert p["path"] == "tiles" and p["splits"] > 1 and not p["stream_k"], (case, p)
    assert plan(STREAM_K)["stream_k"], plan(STREAM_K)
    assert uses_scratch(plan(TRANSPOSED)), plan(TRANSPOSED)
    assert not uses_scratch(plan(NO_SPLIT)), plan(NO_SPLIT)
    # Between them the split cases cover more than one tile configuration.
    assert len({plan(c)["tile"] for c in (SPLIT_A, SPLIT_B, STREAM_K, TRANSPOSED)}) >= 2


@pytest.mark.parametrize("first,second", PAIRS)
def test_two_calls_in_a_row_equal_the_workspace_matmul(dev, orc, first, second):
    from magnetar_hip import ops
    calls = []
    for i, (m, k, n, ta, tb, mode) in enumerate((first, second)):
        a, b, addend = operands(dev, orc, m, k, n, ta, tb, mode, 900 + 10 * i + m % 7)
        da, db = dev.upload(a), dev.upload(b)
        dadd = dev.upload(addend) if addend is not None else None
        print(f"noalloc call {i}: {m}x{k}x{n} ta={ta} tb={tb} mode={mode}", flush=True)
        st, got = noalloc(dev, da, db, m, k, n, ta, tb, dadd, mode)
        assert st == 0, dev_detail()
        calls.append((m, k, n, ta, tb, mode, a, b, addend, da, db, dadd, got))
    # Read both only after the second call has run over the same scratch.
    for m, k, n, ta, tb, mode, a, b, addend, da, db, dadd, got in calls:
        want = ops.matmul(dev, da, db, bool(ta), bool(tb), dadd, mode).numpy()
        assert_bitexact(got.numpy(), want, f"noalloc {m}x{k}x{n}")
        if not ta and not tb:
            for r in np.linspace(0, m - 1, 4).astype(int):
                row = orc.matmul_rows(a, b, int(r), int(r) + 1)
                if mode == 1:
                    row = row + addend
                elif mode == 2:
                    row = row + addend[r:r + 1]
                assert max_normwise_err(got.numpy()[r:r + 1], row) <= TOL


def dev_detail():
    from magnetar_hip import _lib
    return _lib.lib().mhip_last_error_detail().decode()


def test_a_product_beyond_the_scratch_is_refused(dev, orc):
    """3584 x 4096 x 3584 takes 256-tiles split 5 ways over k: 5 partial
    products of 3584^2 floats (257 MB), beyond the 128 MiB array."""
    m = n = 3584
    k = 4096
    a = dev.upload(orc.uniform(m * k, 950, -1.0, 1.0).reshape(m, k))
    b = dev.upload(orc.uniform(k * n, 951, -1.0, 1.0).reshape(k, n))
    st, _ = noalloc(dev, a, b, m, k, n)
    assert st == SHAPE_UNSUPPORTED
    assert "bytes of scratch" in dev_detail()
    # The context works on: a product that fits still runs.
    m2, k2, n2 = SPLIT_A[:3]
    a2 = orc.uniform(m2 * k2, 952, -1.0, 1.0).reshape(m2, k2)
    b2 = orc.uniform(k2 * n2, 953, -1.0, 1.0).reshape(k2, n2)
    st, got = noalloc(dev, dev.upload(a2), dev.upload(b2), m2, k2, n2)
    assert st == 0, dev_detail()
    from magnetar_hip import ops
    assert_bitexact(got.numpy(), ops.matmul(dev, dev.upload(a2), dev.upload(b2)).numpy())


@pytest.mark.parametrize("case", [SPLIT_A, STREAM_K, GEMV])
def test_a_fresh_context_captures_a_split_product_without_allocating(orc, case):
    """A new context has no workspace yet. Inside a capture the ordinary entry
    point would have to grow it, which capturing refuses; the
    allocation-free one needs nothing, and its graph replays equal the eager
    result."""
    import magnetar_hip
    from magnetar_hip import ops
    m, k, n = case[:3]
    a_host = orc.uniform(m * k, 960, -1.0, 1.0).reshape(m, k)
    b_host = orc.uniform(k * n, 961, -1.0, 1.0).reshape(k, n)
    with magnetar_hip.Device(0) as fresh:
        assert uses_scratch(ops.matmul_plan(fresh, m, k, n)), case
        a, b = fresh.upload(a_host), fresh.upload(b_host)
        out = fresh.empty((m, n))
        fresh.sync()
        # The ordinary entry point in a capture on this fresh context: refused.
        fresh.capture_begin()
        with pytest.raises(magnetar_hip.MagnetarHipError) as refused:
            ops.matmul(fresh, a, b, out=out)
        assert refused.value.code == "CaptureUnsupported", refused.value
        with pytest.raises(magnetar_hip.MagnetarHipError):
            fresh.capture_end()
        # The allocation-free one captures.
        fresh.capture_begin()
        st, _ = noalloc(fresh, a, b, m, k, n, out=out)
        assert st == 0, dev_detail()
        graph = fresh.capture_end()
        with magnetar_hip.Device(0) as other:
            want = ops.matmul(other, other.upload(a_host), other.upload(b_host)).numpy()
        for _ in range(3):
            fresh.zeros((m, n))  # eager work between replays
            ops.matmul(fresh, a, b)  # the ordinary entry point, eager: grows the workspace
            graph.launch(0)
            assert_bitexact(out.numpy(), want, "captured noalloc replay")
        graph.close()
