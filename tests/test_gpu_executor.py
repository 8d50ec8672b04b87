"""GPU: the Provider facade and the executor's dispatch contract.

Mirrors the reference's integration tier (src/tests.rs:80-165,
src/tests_hardware_hot_path.rs:134-595): Kernels dispatched by name through
submit_kernel / complete_kernel with Runtime-style attributes; results stay
device-resident between calls; failures keep the overwritten output's value;
errors surface in the reference's categories.
"""
import numpy as np
import pytest

from conftest import assert_bitexact, max_normwise_err, max_rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def provider():
    import magnetar_hip
    p = magnetar_hip.Provider()
    yield p
    p.close()


@pytest.fixture()
def ex(provider):
    ex = provider.execution_api()
    assert ex is not None
    return ex


def inv(kernel, inputs, output, attrs=None, **kw):
    from magnetar_hip import KernelInvocation, TensorRef
    ins = [i if isinstance(i, TensorRef) else TensorRef(i) for i in inputs]
    out = output if isinstance(output, TensorRef) else TensorRef(output)
    return KernelInvocation(kernel, ins, [out], attrs or {}, **kw)


def test_provider_reports_the_device(provider):
    assert provider.health() == "Available"
    devices = provider.devices()
    assert len(devices) == 1
    assert devices[0]["id"] == "hip:0"
    assert devices[0]["memory_capacity"] > 0
    assert "gfx950" in devices[0]["architecture"]
    assert devices[0]["compute_units"] > 0


def test_advertisements(provider):
    adverts = provider.kernel_advertisements()
    names = [a.name for a in adverts]
    assert names == ["matmul", "matmul-bias", "matmul-residual", "silu-mul", "gated-matmul",
                     "embedding", "rmsnorm", "rope", "attention", "softmax", "silu", "add", "mul",
                     "concat", "kv-write", "residual-add", "add-half", "mul-half"]
    by = {a.name: a for a in adverts}
    for name in ("matmul", "rope", "attention", "softmax"):
        assert by[name].rank == 2
    assert by["add-half"].operator_name == "add" and by["mul-half"].operator_name == "mul"
    assert by["add-half"].input_dtypes == [1, 2]
    assert by["add"].input_dtypes == [0]
    assert "rmsnorm-without-weight" in by["rmsnorm"].features
    assert all(a.conformance_profile == "hip-conformance-v1" for a in adverts)
    assert all(a.device_id == "hip:0" for a in adverts)


def test_every_kernel_through_dispatch(ex, orc):
    """One invocation per advertised f32 Kernel, checked against the oracle."""
    rows, hidden, heads, hd, ffn = 8, 64, 4, 16, 96
    x = orc.hashed_values(rows * hidden, 1).reshape(rows, hidden)
    y = orc.hashed_values(rows * hidden, 2).reshape(rows, hidden)
    w = orc.hashed_values(hidden * ffn, 3).reshape(hidden, ffn)
    g = orc.normal(hidden, 4, 1.0, 0.1)
    table = orc.normal(50 * hidden, 5).reshape(50, hidden)
    ids = np.array([3, 0, 49, 7], np.float32)
    for name, arr in dict(x=x, y=y, w=w, g=g, table=table, ids=ids).items():
        ex.write_tensor(name, arr)
    ex.execute(inv("add", ["x", "y"], "o"))
    assert_bitexact(ex.read_tensor("o"), orc.add(x, y)[0])
    ex.execute(inv("residual-add", ["x", "y"], "o"))
    assert_bitexact(ex.read_tensor("o"), orc.add(x, y)[0])
    ex.execute(inv("add", ["x", "g"], "o"))  # bias broadcast
    assert_bitexact(ex.read_tensor("o"), orc.bias_add(x, g)[0])
    ex.execute(inv("mul", ["x", "y"], "o"))
    assert_bitexact(ex.read_tensor("o"), orc.mul(x, y)[0])
    ex.write_tensor("s", np.array([0.25], np.float32))
    ex.execute(inv("mul", ["x", "s"], "o"))  # [1] scalar broadcast
    assert_bitexact(ex.read_tensor("o"), x * np.float32(0.25))
    ex.execute(inv("silu", ["x"], "o"))
    assert max_rel_err(ex.read_tensor("o"), orc.silu(x)[0], 1e-37) <= 1e-6
    ex.execute(inv("silu-mul", ["x", "y"], "o"))
    assert max_rel_err(ex.read_tensor("o"), orc.silu_mul(x, y)[0], 1e-37) <= 1e-6
    ex.execute(inv("softmax", ["x"], "o"))
    assert max_rel_err(ex.read_tensor("o"), orc.softmax_rows(x)[0]) <= 1e-4
    ex.execute(inv("rmsnorm", ["x", "g"], "o", {"epsilon": 1e-5}))
    assert max_rel_err(ex.read_tensor("o"), orc.rmsnorm(x, g, 1e-5)[0]) <= 1e-4
    ex.execute(inv("rmsnorm", ["x"], "o"))  # no weight, default epsilon 1e-6
    assert max_rel_err(ex.read_tensor("o"), orc.rmsnorm(x, None, 1e-6)[0]) <= 1e-4
    ex.execute(inv("rmsnorm", ["x"], "o",
                   {"head_count": heads, "head_dimension": hd}))
    assert max_rel_err(ex.read_tensor("o"), orc.rmsnorm(x, None, 1e-6, cols=hd)[0]) <= 1e-4
    ex.execute(inv("embedding", ["table", "ids"], "o"))
    assert_bitexact(ex.read_tensor("o"), table[[3, 0, 49, 7]])
    ex.execute(inv("embedding", ["table", "ids"], "o", {"scale": 8.0}))
    assert_bitexact(ex.read_tensor("o"), table[[3, 0, 49, 7]] * np.float32(8.0))
    ex.execute(inv("matmul", ["x", "w"], "o"))
    assert max_normwise_err(ex.read_tensor("o"), orc.matmul(x, w)[0]) <= 1e-4
    ex.write_tensor("bias", orc.hashed_values(ffn, 6))
    ex.execute(inv("matmul-bias", ["x", "w", "bias"], "o"))
    plain = orc.matmul(x, w)[0]
    assert max_normwise_err(ex.read_tensor("o"), plain + orc.hashed_values(ffn, 6)) <= 1e-4
    ex.write_tensor("w2", orc.hashed_values(hidden * ffn, 7).reshape(hidden, ffn))
    ex.execute(inv("gated-matmul", ["x", "w", "w2"], "o"))
    gate = orc.matmul(x, w)[0]
    up = orc.matmul(x, orc.hashed_values(hidden * ffn, 7).reshape(hidden, ffn))[0]
    assert max_normwise_err(ex.read_tensor("o"), orc.silu_mul(gate, up)[0]) <= 1e-4
    ex.execute(inv("rope", ["x"], "o", {"dimension": hd, "head_count": heads,
                                        "position_offset": 5}))
    want, _ = orc.rope(x, orc.rope_params(hd, heads, position_offset=5))
    assert np.max(np.abs(ex.read_tensor("o") - want)) <= 1e-6
    ex.execute(inv("attention", ["x", "y", "x"], "o", {"head_count": heads, "head_dimension": hd,
                                                       "causal": True}))
    want, _ = orc.attention(x, y, x, orc.attention_params(rows, rows, heads, hd, causal=True))
    assert max_normwise_err(ex.read_tensor("o"), want) <= 1e-4
    ex.execute(inv("concat", ["x", "y"], "o"))
    assert_bitexact(ex.read_tensor("o"), np.concatenate([x, y]))


def test_device_resident_chain(ex, orc):
    """weight -> matmul -> rmsnorm -> rope -> projection, never leaving the
    device (src/tests_hardware_hot_path.rs:339-526), against the CPU chain."""
    seq, hidden, heads = 32, 256, 4
    x = orc.normal(seq * hidden, 11, 0.0, 1.0).reshape(seq, hidden)
    wq = orc.normal(hidden * hidden, 12, 0.0, 0.02).reshape(hidden, hidden)
    wo = orc.normal(hidden * hidden, 13, 0.0, 0.02).reshape(hidden, hidden)
    gain = np.ones(hidden, np.float32)
    for name, arr in dict(x=x, wq=wq, wo=wo, gain=gain).items():
        ex.write_tensor(name, arr)
    ex.execute(inv("matmul", ["x", "wq"], "q"))
    ex.execute(inv("rmsnorm", ["q", "gain"], "qn", {"epsilon": 1e-5}))
    ex.execute(inv("rope", ["qn"], "qr", {"dimension": 64, "head_count": heads}))
    ex.execute(inv("matmul", ["qr", "wo"], "out"))
    q, _ = orc.matmul(x, wq)
    qn, _ = orc.rmsnorm(q, gain, 1e-5)
    qr, _ = orc.rope(qn, orc.rope_params(64, heads))
    want, _ = orc.matmul(qr, wo)
    assert max_normwise_err(ex.read_tensor("out"), want) <= 1e-4
    assert ex.resident_shape("out") == ((seq, hidden), 0)
    rows = ex.read_tensor_rows("out", 5, 3)
    assert_bitexact(rows, ex.read_tensor("out")[5:8])


def test_attribute_errors(ex):
    from magnetar_hip import KernelError, Integer, String, DType, F16
    ex.write_tensor("a", np.ones((4, 8), np.float32))
    ex.write_tensor("b", np.ones((8, 4), np.float32))
    cases = [
        (inv("rope", ["a"], "o", {}), "KernelAttributeUnsupported"),  # dimension required
        (inv("rope", ["a"], "o", {"dimension": 4, "position_offset": Integer(-1)}), "KernelAttributeUnsupported"),
        (inv("rope", ["a"], "o", {"dimension": 4, "position_offset": "3"}), "KernelAttributeUnsupported"),
        (inv("rope", ["a"], "o", {"dimension": 4, "rotation_pairing": "neox"}), "KernelAttributeUnsupported"),
        (inv("rope", ["a"], "o", {"dimension": 4, "position_mode": "explicit"}), "KernelAttributeUnsupported"),
        (inv("rope", ["a"], "o", {"dimension": 4, "partial_rotary_factor": 1.5}), "KernelAttributeUnsupported"),
        (inv("rope", ["a"], "o", {"dimension": 5}), "KernelShapeUnsupported"),
        (inv("attention", ["a", "a", "a"], "o", {"head_dimension": 8}), "KernelAttributeUnsupported"),
        (inv("attention", ["a", "a", "a"], "o", {"head_count": 1, "head_dimension": 8,
                                                "attention_mask_kind": "causal"}), "KernelAttributeUnsupported"),
        (inv("attention", ["a", "a", "a"], "o", {"head_count": 1, "head_dimension": 8,
                                                "window_size": 4}), "KernelShapeUnsupported"),
        (inv("attention", ["a", "a", "a"], "o", {"head_count": 1, "head_dimension": 8,
                                                "scale": Integer(2)}), "KernelAttributeUnsupported"),
        (inv("rmsnorm", ["a", "a"], "o", {"with_scale": False}), "KernelAttributeUnsupported"),
        (inv("rmsnorm", ["a"], "o", {"head_count": 2}), "KernelAttributeUnsupported"),
        (inv("rmsnorm", ["a"], "o", {"epsilon": -1.0}), "KernelShapeUnsupported"),
        (inv("matmul", ["a", "b"], "o", {"accumulation_dtype": DType(F16)}), "KernelDTypeUnsupported"),
        (inv("matmul", ["a", "a"], "o"), "KernelShapeUnsupported"),
        (inv("mul", ["a", "b"], "o"), "KernelShapeUnsupported"),
        (inv("add", ["a", "b"], "o"), "KernelShapeUnsupported"),
        (inv("no-such-kernel", ["a"], "o"), "KernelNotFound"),
        (inv("add", ["a", "missing"], "o"), "KernelExecutionFailed"),
        (inv("embedding", ["a", "a"], "o", {"scale": Integer(3)}), "KernelAttributeUnsupported"),
    ]
    for invocation, code in cases:
        with pytest.raises(KernelError) as err:
            ex.execute(invocation)
        assert err.value.code == code, (invocation.kernel, invocation.attributes, err.value)


def test_deadline_zero_times_out(ex):
    from magnetar_hip import KernelError
    ex.write_tensor("a", np.ones(4, np.float32))
    with pytest.raises(KernelError) as err:
        ex.execute(inv("silu", ["a"], "o", deadline_millis=0))
    assert err.value.code == "KernelTimeout"
    kinds = [o[0] for o in ex.observations()[-2:]]
    assert kinds == ["KernelDispatchStarted", "KernelTimeout"]


def test_failed_dispatch_keeps_the_output_value(ex):
    """src/tests_hardware_hot_path.rs:261-330: a failing invocation whose
    output resource already holds a value leaves that value in place."""
    from magnetar_hip import KernelError
    ex.write_tensor("a", np.arange(6, dtype=np.float32).reshape(2, 3))
    ex.write_tensor("bad", np.arange(4, dtype=np.float32).reshape(2, 2))
    ex.write_tensor("keep", np.full((2, 3), 7.0, np.float32))
    with pytest.raises(KernelError):
        ex.execute(inv("add", ["a", "bad"], "keep"))
    assert_bitexact(ex.read_tensor("keep"), np.full((2, 3), 7.0, np.float32))
    # An invalid embedding id fails through the device flag, also keeping the value.
    ex.write_tensor("table", np.zeros((4, 3), np.float32))
    ex.write_tensor("ids", np.array([9.0], np.float32))
    with pytest.raises(KernelError) as err:
        ex.execute(inv("embedding", ["table", "ids"], "keep"))
    assert err.value.code == "KernelShapeUnsupported"
    assert "valid in-range" in err.value.detail
    assert_bitexact(ex.read_tensor("keep"), np.full((2, 3), 7.0, np.float32))
    # The same resource overwritten successfully reuses or replaces it.
    ex.execute(inv("add", ["a", "a"], "keep"))
    assert_bitexact(ex.read_tensor("keep"), np.arange(6, dtype=np.float32).reshape(2, 3) * 2)


def test_output_reading_its_own_input(ex):
    ex.write_tensor("acc", np.ones((3, 4), np.float32))
    ex.write_tensor("one", np.ones((3, 4), np.float32))
    for _ in range(3):
        ex.execute(inv("add", ["acc", "one"], "acc"))
    assert_bitexact(ex.read_tensor("acc"), np.full((3, 4), 4.0, np.float32))


def test_softmax_without_finite_entry_fails(ex):
    from magnetar_hip import KernelError
    ex.write_tensor("m", np.full((2, 3), -np.inf, np.float32))
    with pytest.raises(KernelError) as err:
        ex.execute(inv("softmax", ["m"], "o"))
    assert err.value.code == "KernelExecutionFailed"


@pytest.mark.parametrize("dtype", [1, 2])
def test_half_kernels_through_dispatch(ex, orc, dtype):
    """add-half / mul-half on 2-byte resident tensors, bit-exact against the
    reference's model (src/tests_hardware_hot_path.rs:539-626)."""
    from magnetar_hip import TensorRef
    a = orc.normal(1000, 21)
    b = orc.normal(1000, 22)
    ha, hb = orc.encode_half(a, dtype - 1), orc.encode_half(b, dtype - 1)
    ex.write_tensor("ha", ha, dtype)
    ex.write_tensor_values("hb", b, dtype)  # encoded on the device
    assert_bitexact(ex.read_tensor("hb"), hb)
    for kernel, op in (("add-half", "add"), ("mul-half", "mul")):
        ex.execute(inv(kernel, [TensorRef("ha", (1000,), dtype), TensorRef("hb", (1000,), dtype)],
                       TensorRef("ho", (1000,), dtype)))
        got = ex.read_tensor("ho")
        assert got.dtype == np.uint16
        assert_bitexact(got, orc.half_binary(ha, hb, dtype - 1, op))
        assert_bitexact(ex.read_tensor_values("ho"), orc.decode_half(got, dtype - 1))
    # f32-stored operands are encoded on the device, as the reference encodes on upload.
    ex.write_tensor("fa", a)
    ex.execute(inv("add-half", [TensorRef("fa", (1000,), dtype), TensorRef("hb", (1000,), dtype)],
                   TensorRef("ho", (1000,), dtype)))
    assert_bitexact(ex.read_tensor("ho"), orc.half_binary(ha, hb, dtype - 1, "add"))


def test_half_kernel_rejects_f32_dtype(ex):
    from magnetar_hip import KernelError, TensorRef
    ex.write_tensor("fa", np.ones(4, np.float32))
    with pytest.raises(KernelError) as err:
        ex.execute(inv("add-half", [TensorRef("fa"), TensorRef("fa")], TensorRef("o")))
    assert err.value.code == "KernelDTypeUnsupported"


def test_observations_and_release(ex):
    ex.write_tensor("r", np.ones(8, np.float32))
    ex.execute(inv("silu", ["r"], "r2", id="obs-1"))
    obs = ex.observations()
    assert obs[-2][:3] == ("KernelDispatchStarted", "silu", "obs-1")
    assert obs[-1][:3] == ("KernelDispatchCompleted", "silu", "obs-1")
    n = ex.tensor_count()
    ex.release_tensor("r2")
    assert ex.tensor_count() == n - 1
    ex.copy_tensor("r", "r3")
    assert_bitexact(ex.read_tensor("r3"), np.ones(8, np.float32))


def test_kv_write_through_the_executor(ex):
    """kv-write (src/executor.rs:1366-1420): in place when the output is the
    store, into a copy otherwise; a failed write leaves the store's rows."""
    from magnetar_hip import KernelError, Integer
    from magnetar_hip.executor import KV_F32, KV_TQ4
    assert ex.write_zeroed_kv_store("kv", (4, 2), KV_F32, 2)
    ex.write_tensor("kv_rows", np.array([[1, 2], [3, 4]], np.float32))
    ex.execute(inv("kv-write", ["kv", "kv_rows"], "kv", {"row_offset": Integer(1)}))
    assert ex.read_tensor("kv").ravel().tolist() == [0, 0, 1, 2, 3, 4, 0, 0]
    ex.execute(inv("kv-write", ["kv", "kv_rows"], "kv_copy", {"row_offset": Integer(2)}))
    assert ex.read_tensor("kv_copy").ravel().tolist() == [0, 0, 1, 2, 1, 2, 3, 4]
    assert ex.read_tensor("kv").ravel().tolist() == [0, 0, 1, 2, 3, 4, 0, 0]
    ex.write_tensor("kv_wide", np.ones((1, 3), np.float32))
    cases = [
        (inv("kv-write", ["kv", "kv_rows"], "kv", {"row_offset": Integer(3)}), "KernelShapeUnsupported"),
        (inv("kv-write", ["kv", "kv_rows"], "kv", {}), "KernelAttributeUnsupported"),
        (inv("kv-write", ["kv", "kv_rows"], "kv", {"row_offset": Integer(-1)}), "KernelAttributeUnsupported"),
        (inv("kv-write", ["kv", "kv_wide"], "kv", {"row_offset": Integer(0)}), "KernelShapeUnsupported"),
        (inv("kv-write", ["kv", "nothing"], "kv", {"row_offset": Integer(0)}), "KernelExecutionFailed"),
        (inv("kv-write", ["nothing", "kv_rows"], "kv", {"row_offset": Integer(0)}), "KernelExecutionFailed"),
    ]
    for invocation, code in cases:
        with pytest.raises(KernelError) as err:
            ex.execute(invocation)
        assert err.value.code == code, (invocation.attributes, err.value)
        assert ex.read_tensor("kv").ravel().tolist() == [0, 0, 1, 2, 3, 4, 0, 0]
    # The quantized stores are declined, and nothing is written.
    assert not ex.write_zeroed_kv_store("kv_tq", (4, 2), KV_TQ4, 2)
    with pytest.raises(KernelError):
        ex.read_tensor("kv_tq")


@pytest.mark.parametrize("rows", [1, 3, 8, 16, 40])
def test_gated_matmul_is_bit_identical_to_its_parts(ex, orc, rows):
    """gated-matmul equals matmul, matmul and silu-mul dispatched separately,
    bit for bit (src/tests_conformance.rs:486-565): decode rows take the fused
    GEMV set, 40 rows the separate kernels; also into an offered output
    buffer of the right size."""
    hidden, ffn = 256, 344
    ex.write_tensor("g.x", orc.hashed_values(rows * hidden, 11 + rows).reshape(rows, hidden))
    ex.write_tensor("g.w", orc.hashed_values(hidden * ffn, 12).reshape(hidden, ffn))
    ex.write_tensor("g.u", orc.hashed_values(hidden * ffn, 13).reshape(hidden, ffn))
    ex.execute(inv("matmul", ["g.x", "g.w"], "g.gate"))
    ex.execute(inv("matmul", ["g.x", "g.u"], "g.up"))
    ex.execute(inv("silu-mul", ["g.gate", "g.up"], "g.want"))
    want = ex.read_tensor("g.want")
    ex.execute(inv("gated-matmul", ["g.x", "g.w", "g.u"], "g.out"))
    assert_bitexact(ex.read_tensor("g.out"), want)
    ex.execute(inv("gated-matmul", ["g.x", "g.w", "g.u"], "g.out"))  # offered buffer
    assert_bitexact(ex.read_tensor("g.out"), want)
    for name in ("g.x", "g.w", "g.u", "g.gate", "g.up", "g.want", "g.out"):
        ex.release_tensor(name)


def _bf16_exact(values):
    return (values.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


@pytest.mark.parametrize("m,k,n,ta,tb,path", [
    (24, 300, 512, False, False, "small_tiles"),
    (16, 1100, 512, False, False, "gemv_row_blocks"),
    (40, 4096, 4096, False, False, "splits"),
    (200, 2050, 1900, False, False, "stream_k"),
    (400, 1024, 1900, False, True, "splits"),
    (130, 512, 1901, True, True, "splits"),      # odd n: the scalar reduction
    (4000, 64, 4064, False, True, "tiles"),
    (301, 257, 203, True, False, None),
])
def test_gated_matmul_on_every_matmul_path(ex, dev, orc, m, k, n, ta, tb, path):
    """Up to 32 rows of small products take the GEMV set (on one-launch
    small MFMA tiles or row blocks of 8, as the matmul would); other shapes
    run the gate product, then the up product with silu(gate) applied to
    each finished sum: on every kernel path of the matmul (whole-k splits,
    stream-K, direct tile stores; the path is asserted) and with transposes.
    Each is bit-identical to matmul, matmul and silu-mul dispatched
    separately; then again with a compact bf16 up weight against its
    widened f32 form."""
    from magnetar_hip import Boolean, ops
    plan = ops.matmul_plan(dev, m, k, n, ta, tb)
    if path in ("gemv_row_blocks", "small_tiles"):
        assert plan["path"] == path, plan
    elif path is not None:
        assert plan["path"] == "tiles", plan
        assert (path == "stream_k") == bool(plan["stream_k"]), plan
        assert (path == "splits") == (plan["splits"] > 1), plan
    attrs = {"transpose_a": Boolean(ta), "transpose_b": Boolean(tb)}
    x = orc.hashed_values(m * k, 21 + m).reshape((k, m) if ta else (m, k))
    wg = orc.hashed_values(k * n, 22 + n).reshape((n, k) if tb else (k, n))
    wu = _bf16_exact(orc.hashed_values(k * n, 23 + n)).reshape(wg.shape)
    ex.write_tensor("gp.x", x)
    ex.write_tensor("gp.g", wg)
    ex.write_tensor("gp.u", wu)
    ex.execute(inv("matmul", ["gp.x", "gp.g"], "gp.gate", attrs))
    ex.execute(inv("matmul", ["gp.x", "gp.u"], "gp.up", attrs))
    ex.execute(inv("silu-mul", ["gp.gate", "gp.up"], "gp.want"))
    want = ex.read_tensor("gp.want")
    ex.execute(inv("gated-matmul", ["gp.x", "gp.g", "gp.u"], "gp.out", attrs))
    got = ex.read_tensor("gp.out")
    print(f"[{m},{k},{n}] ta={ta} tb={tb}: {plan}")
    assert_bitexact(got, want)
    if ex.write_weight_tensor("gp.uc", wu):
        ex.execute(inv("gated-matmul", ["gp.x", "gp.g", "gp.uc"], "gp.outc", attrs))
        assert_bitexact(ex.read_tensor("gp.outc"), want)
        ex.release_tensor("gp.uc")
        ex.release_tensor("gp.outc")
    for name in ("gp.x", "gp.g", "gp.u", "gp.gate", "gp.up", "gp.want", "gp.out"):
        ex.release_tensor(name)


def test_out_of_device_memory_is_triggered_by_a_real_over_capacity_allocation(dev, ex):
    """src/tests.rs:47-71: an allocation of 64x the device's total memory
    fails as OutOfDeviceMemory (mapped as src/error.rs:97-133); through the
    executor the same failure is KernelOutOfDeviceMemory. Both leave the
    context usable."""
    import ctypes
    from magnetar_hip import KernelError, _lib
    total = dev.info()["total_memory"]
    ptr = ctypes.c_void_p()
    st = _lib.lib().mhip_alloc(dev.ctx, total * 64, ctypes.byref(ptr))
    assert st == 5 and not ptr.value  # MHIP_OUT_OF_DEVICE_MEMORY
    assert _lib.lib().mhip_status_name(st).decode() == "OutOfDeviceMemory"
    assert "device bytes" in _lib.lib().mhip_last_error_detail().decode()
    with pytest.raises(KernelError) as err:
        ex.write_zeroed_tensor("oom.impossible", (total * 64 // 4,))
    assert err.value.code == "KernelOutOfDeviceMemory"
    # The context still allocates and runs.
    ex.write_tensor("oom.after", np.arange(8, dtype=np.float32).reshape(2, 4))
    ex.execute(inv("silu", ["oom.after"], "oom.after.silu"))
    assert ex.read_tensor("oom.after.silu").shape == (2, 4)
    st = _lib.lib().mhip_alloc(dev.ctx, 1024, ctypes.byref(ptr))
    assert st == 0 and ptr.value
    _lib.check(_lib.lib().mhip_free(dev.ctx, ptr))


def test_deferred_checks_report_at_the_next_read(ex, orc):
    """With deferred checks an invalid embedding id or an all -inf softmax row
    no longer fails its dispatch: the next read (or check()) raises it in the
    same category, naming the first unchecked dispatch; valid chains give the
    same bits as with the reference's per-dispatch checks."""
    from magnetar_hip import KernelError, KernelInvocation, TensorRef
    table = orc.normal(16 * 8, 71).reshape(16, 8)
    ex.write_tensor("table", table)
    ex.write_tensor("ids", np.array([3.0, 15.0, 0.0], np.float32))
    ex.write_tensor("bad", np.array([2.0, 16.0], np.float32))
    ex.write_tensor("m", np.full((2, 3), -np.inf, np.float32))
    ex.execute(inv("embedding", ["table", "ids"], "e"))
    ex.execute(inv("softmax", ["e"], "p"))
    eager = ex.read_tensor("p")
    ex.set_deferred_checks(True)
    try:
        ex.execute(inv("embedding", ["table", "ids"], "e2"))
        ex.execute(inv("softmax", ["e2"], "p2"))
        assert_bitexact(ex.read_tensor("p2"), eager)
        ex.execute(KernelInvocation("embedding", [TensorRef("table"), TensorRef("bad")],
                                    [TensorRef("e3")], {}, id="lookup-7"))
        ex.execute(inv("softmax", ["e"], "p3"))  # valid, shares the check
        with pytest.raises(KernelError) as err:
            ex.read_tensor("p3")
        assert err.value.code == "KernelShapeUnsupported"
        assert "valid in-range" in err.value.detail
        assert "2 dispatch(es)" in err.value.detail and "lookup-7" in err.value.detail
        assert_bitexact(ex.read_tensor("p3"), eager)  # reported once, then clear
        ex.execute(inv("softmax", ["m"], "p4"))
        with pytest.raises(KernelError) as err:
            ex.check()
        assert err.value.code == "KernelExecutionFailed"
        ex.check()
        ex.execute(inv("softmax", ["m"], "p4"))
        with pytest.raises(KernelError) as err:
            ex.select_greedy_column("p3")
        assert err.value.code == "KernelExecutionFailed"
        assert ex.select_greedy_column("p3", 1) == int(np.argmax(eager[1]))
        ex.execute(inv("embedding", ["table", "bad"], "e3"))
        with pytest.raises(KernelError):  # disabling checks what is pending
            ex.set_deferred_checks(False)
    finally:
        try:
            ex.set_deferred_checks(False)
        except KernelError:
            pass
    with pytest.raises(KernelError):
        ex.execute(inv("embedding", ["table", "bad"], "e3"))
