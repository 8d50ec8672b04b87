"""GPU: step capture and replay (reference src/executor.rs:177-336,
src/kernels.rs:1019-1349; tests src/tests_hardware_hot_path.rs:633-833).

A captured step is a HIP graph of the context's stream. Replays with an
offset move every advancing attribute (RoPE position_offset, attention
key_count, kv-write row_offset) by it, and must equal the same invocations
dispatched eagerly at the advanced values, bit for bit. Each graph is replayed
several times with eager work and synchronisation in between, and every replay
is checked.
"""
import numpy as np
import pytest

from conftest import max_normwise_err, max_rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def provider():
    import magnetar_hip
    p = magnetar_hip.Provider()
    yield p
    p.close()


@pytest.fixture()
def ex(provider):
    return provider.execution_api()


def inv(kernel, inputs, output, attrs=None):
    from magnetar_hip import KernelInvocation, TensorRef
    return KernelInvocation(kernel, [TensorRef(i) for i in inputs], [TensorRef(output)], attrs or {})


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_the_executor_supports_step_capture(ex):
    assert ex.supports_step_capture()


def test_a_captured_step_replays_with_an_advanced_position(ex, orc):
    """src/tests_hardware_hot_path.rs:633-727: rope then rmsnorm, captured at
    position 3 and replayed at offset 4 with other inputs, equals the eager
    step at position 7."""
    from magnetar_hip import Integer, KernelError
    first = np.array([[0.5, -1.0, 2.0, 0.25], [1.5, 3.0, -0.75, 1.0]], np.float32)
    second = np.array([[-2.0, 0.5, 1.0, 4.0], [0.0, -1.5, 2.5, 0.75]], np.float32)
    ex.write_tensor("replay.norm.weight", np.array([0.5, 1.0, 1.5, 2.0], np.float32))

    def step(position, read=True):
        ex.execute(inv("rope", ["replay.x"], "replay.rope.out",
                       {"base": 10000.0, "dimension": 4, "position_offset": Integer(position)}))
        ex.execute(inv("rmsnorm", ["replay.rope.out", "replay.norm.weight"], "replay.sum.out",
                       {"epsilon": 1e-6}))
        return ex.read_tensor("replay.sum.out") if read else None

    ex.write_tensor("replay.x", second)
    second_at_7 = step(7)
    ex.write_tensor("replay.x", first)
    first_at_3 = step(3)
    assert not np.array_equal(first_at_3, second_at_7)
    # The oracle's step at each position.
    gain = np.array([0.5, 1.0, 1.5, 2.0], np.float32)
    for x, position, got in ((first, 3, first_at_3), (second, 7, second_at_7)):
        rotated, _ = orc.rope(x, orc.rope_params(4, 1, position_offset=position))
        want, _ = orc.rmsnorm(rotated, gain, 1e-6)
        assert max_rel_err(got, want) <= 1e-4, position

    ex.begin_step_capture(["position_offset"])
    step(3, read=False)
    capture = ex.end_step_capture()
    assert capture.endswith(":step-capture:" + capture.rsplit(":", 1)[1])
    assert np.array_equal(bits(ex.read_tensor("replay.sum.out")), bits(first_at_3))
    for _ in range(3):
        ex.replay_step(capture, 4, {"replay.x": second})
        assert np.array_equal(bits(ex.read_tensor("replay.sum.out")), bits(second_at_7))
        ex.replay_step(capture, 0, {"replay.x": first})
        assert np.array_equal(bits(ex.read_tensor("replay.sum.out")), bits(first_at_3))

    # A fresh upload gives the input another buffer.
    ex.write_tensor("replay.x", first)
    with pytest.raises(KernelError) as err:
        ex.replay_step(capture, 0, {"replay.x": first})
    assert err.value.code == "StepReplayInvalidated"
    ex.release_step_capture(capture)
    with pytest.raises(KernelError) as err:
        ex.replay_step(capture, 0, {})
    assert err.value.code == "StepReplayInvalidated"

    # A host upload cannot be captured: the capture fails, the stream works.
    ex.begin_step_capture(["position_offset"])
    with pytest.raises(KernelError):
        ex.write_tensor("replay.x", first)
    with pytest.raises(KernelError) as err:
        ex.end_step_capture()
    assert "cannot be captured" in err.value.detail
    assert np.array_equal(bits(step(3)), bits(first_at_3))


def test_capture_refuses_what_it_cannot_replay(ex):
    from magnetar_hip import KernelError
    ex.write_tensor("cap.a", np.ones((2, 8), np.float32))
    ex.execute(inv("softmax", ["cap.a"], "cap.s"))
    ex.begin_step_capture([])
    with pytest.raises(KernelError):
        ex.begin_step_capture([])          # one capture at a time
    with pytest.raises(KernelError):
        ex.execute(inv("softmax", ["cap.a"], "cap.s"))
    with pytest.raises(KernelError) as err:
        ex.end_step_capture()
    assert "softmax cannot be captured" in err.value.detail
    # A fresh output needs an allocation, which cannot be captured either.
    ex.begin_step_capture([])
    with pytest.raises(KernelError):
        ex.execute(inv("silu", ["cap.a"], "cap.new_output"))
    ex.abort_step_capture()
    with pytest.raises(KernelError):
        ex.end_step_capture()               # nothing in progress
    ex.execute(inv("silu", ["cap.a"], "cap.new_output"))
    assert ex.read_tensor("cap.new_output").shape == (2, 8)


def test_a_captured_gated_matmul_survives_a_larger_eager_one(ex, orc):
    """gated-matmul's matmul path keeps the gate product in a buffer the
    executor reuses and grows. A larger eager call grows it after a step was
    captured; the buffer the graph recorded stays valid, so replays (with
    other inputs, eager calls in between) still equal the eager results bit
    for bit."""
    m, k, n = 40, 256, 344
    x1 = orc.hashed_values(m * k, 31).reshape(m, k)
    x2 = orc.hashed_values(m * k, 32).reshape(m, k)
    ex.write_tensor("cg.w", orc.hashed_values(k * n, 33).reshape(k, n))
    ex.write_tensor("cg.u", orc.hashed_values(k * n, 34).reshape(k, n))

    def step():
        ex.execute(inv("gated-matmul", ["cg.x", "cg.w", "cg.u"], "cg.out"))

    def larger():
        ex.execute(inv("gated-matmul", ["cg.bx", "cg.bw", "cg.bu"], "cg.bout"))
        return ex.read_tensor("cg.bout")

    ex.write_tensor("cg.x", x2)
    step()
    want2 = ex.read_tensor("cg.out")
    ex.write_tensor("cg.x", x1)
    step()
    want1 = ex.read_tensor("cg.out")
    assert not np.array_equal(bits(want1), bits(want2))
    ex.begin_step_capture([])
    step()
    capture = ex.end_step_capture()
    big_m, big_k, big_n = 400, 1024, 1900
    ex.write_tensor("cg.bx", orc.hashed_values(big_m * big_k, 35).reshape(big_m, big_k))
    ex.write_tensor("cg.bw", orc.hashed_values(big_k * big_n, 36).reshape(big_k, big_n))
    ex.write_tensor("cg.bu", orc.hashed_values(big_k * big_n, 37).reshape(big_k, big_n))
    big = larger()
    for _ in range(3):
        ex.replay_step(capture, 0, {"cg.x": x2})
        assert np.array_equal(bits(ex.read_tensor("cg.out")), bits(want2))
        assert np.array_equal(bits(larger()), bits(big))
        ex.replay_step(capture, 0, {"cg.x": x1})
        assert np.array_equal(bits(ex.read_tensor("cg.out")), bits(want1))
    ex.release_step_capture(capture)
    for name in ("cg.x", "cg.w", "cg.u", "cg.out", "cg.bx", "cg.bw", "cg.bu", "cg.bout"):
        ex.release_tensor(name)


def _values(count, seed):
    """The reference test's generator (src/tests_hardware_hot_path.rs:752-756)."""
    i = np.arange(count, dtype=np.int64)
    return ((((i * 37 + seed * 11) % 97).astype(np.float32) - 48.0) / 64.0).astype(np.float32)


@pytest.mark.parametrize("rows,head_dimension", [(16, 64), (32, 128), (8, 64)])
def test_a_captured_prefill_attention_replays_at_its_key_count(ex, orc, rows, head_dimension):
    """src/tests_hardware_hot_path.rs:729-827: several query rows replay with new
    queries exactly like an eager dispatch, and only at offset 0."""
    from magnetar_hip import Integer, KernelError
    width = 2 * head_dimension
    capacity = 4 * rows
    pre = f"prefill-attention.{rows}.{head_dimension}"
    first = _values(rows * width, 1).reshape(rows, width)
    second = _values(rows * width, 2).reshape(rows, width)
    ex.write_tensor(pre + ".k", _values(capacity * width, 3).reshape(capacity, width))
    ex.write_tensor(pre + ".v", _values(capacity * width, 4).reshape(capacity, width))
    attrs = {"head_count": Integer(2), "head_dimension": Integer(head_dimension), "causal": True,
             "key_count": Integer(rows)}

    def attention():
        ex.execute(inv("attention", [pre + ".q", pre + ".k", pre + ".v"], pre + ".out", attrs))

    ex.write_tensor(pre + ".q", second)
    attention()
    expected_second = ex.read_tensor(pre + ".out")
    ex.write_tensor(pre + ".q", first)
    attention()
    expected_first = ex.read_tensor(pre + ".out")
    assert not np.array_equal(expected_first, expected_second)
    k_host = _values(capacity * width, 3).reshape(capacity, width)
    v_host = _values(capacity * width, 4).reshape(capacity, width)
    ap = orc.attention_params(rows, capacity, 2, head_dimension, causal=True, key_count=rows)
    for q_host, got in ((first, expected_first), (second, expected_second)):
        want, st = orc.attention(q_host, k_host, v_host, ap)
        assert st == 0
        assert max_normwise_err(got, want) <= 1e-4

    ex.begin_step_capture(["key_count"])
    attention()
    capture = ex.end_step_capture()
    assert np.array_equal(bits(ex.read_tensor(pre + ".out")), bits(expected_first))
    for _ in range(2):
        ex.replay_step(capture, 0, {pre + ".q": second})
        assert np.array_equal(bits(ex.read_tensor(pre + ".out")), bits(expected_second))
        ex.replay_step(capture, 0, {pre + ".q": first})
        assert np.array_equal(bits(ex.read_tensor(pre + ".out")), bits(expected_first))
    with pytest.raises(KernelError) as err:
        ex.replay_step(capture, 1, {pre + ".q": first})
    assert err.value.code == "StepReplayInvalidated"
    ex.release_step_capture(capture)


def _rope_pair_err(got, want):
    """Largest |got - want| over each rotated pair, relative to the pair's norm
    (RoPE's bar: a rotation keeps the pair's norm, whatever its angle)."""
    g = np.asarray(got, np.float64).reshape(-1, 2)
    w = np.asarray(want, np.float64).reshape(-1, 2)
    norm = np.maximum(np.hypot(w[:, 0], w[:, 1]), 1e-30)
    return float(np.max(np.hypot(*(g - w).T) / norm)) if g.size else 0.0


DECODE_CASES = [
    # heads, kv_heads, dim, first position, capacity, replay offsets
    (4, 4, 64, 0, 40, (0, 1, 2, 3, 4, 5)),
    (8, 2, 128, 0, 40, (0, 1, 2, 3, 4, 5)),
    (2, 1, 4, 0, 40, (0, 1, 2, 3, 4, 5)),
    # More than 8 query heads per KV head, captured past 256 keys and replayed
    # far past the captured count (keys the capture-time split never saw).
    (32, 2, 128, 300, 512, (0, 1, 37, 100, 180, 211)),
    (16, 1, 64, 260, 640, (0, 5, 120, 379)),
    (12, 1, 128, 257, 400, (0, 64, 142)),
    # A store large enough for the double-length key chunks (chosen from the
    # capacity, so the eager steps and the capture split the keys alike).
    (32, 32, 128, 2000, 8200, (0, 7, 900)),
]


@pytest.mark.parametrize("heads,kv_heads,dim,start,capacity,offsets", DECODE_CASES)
def test_a_captured_decode_step_advances_position_cache_row_and_key_count(
        ex, orc, heads, kv_heads, dim, start, capacity, offsets):
    """A decode step -- RoPE on q and k at position p, kv-write of k and v at row
    p, attention over key_count p + 1 -- captured at p = start and replayed at
    offset t equals the eager step at p = start + t (outputs and cache rows,
    bit for bit) and the oracle's step at that position: RoPE at p + t, the
    rows written into a host copy of the cache, attention over the cache's
    first p + t + 1 rows."""
    from magnetar_hip import Integer
    qw, kw = heads * dim, kv_heads * dim
    pre = f"dec.{heads}.{kv_heads}.{dim}.{start}"
    n = len(offsets)
    q_in = [orc.normal(qw, 10 + t).reshape(1, qw) for t in range(n)]
    k_in = [orc.normal(kw, 30 + t).reshape(1, kw) for t in range(n)]
    v_in = [orc.normal(kw, 50 + t).reshape(1, kw) for t in range(n)]
    history_k = np.zeros((capacity, kw), np.float32)
    history_v = np.zeros((capacity, kw), np.float32)
    history_k[:start] = orc.normal(start * kw, 70, 0.0, 0.5).reshape(start, kw)
    history_v[:start] = orc.normal(start * kw, 71, 0.0, 0.5).reshape(start, kw)

    def stores():
        if start:
            ex.write_tensor(pre + ".kc", history_k)
            ex.write_tensor(pre + ".vc", history_v)
        else:
            assert ex.write_zeroed_kv_store(pre + ".kc", (capacity, kw))
            assert ex.write_zeroed_kv_store(pre + ".vc", (capacity, kw))

    def step(p, read=True):
        rope = {"dimension": Integer(dim), "position_offset": Integer(p)}
        ex.execute(inv("rope", [pre + ".q"], pre + ".qr", dict(rope, head_count=Integer(heads))))
        ex.execute(inv("rope", [pre + ".k"], pre + ".kr", dict(rope, head_count=Integer(kv_heads))))
        ex.execute(inv("kv-write", [pre + ".kc", pre + ".kr"], pre + ".kc", {"row_offset": Integer(p)}))
        ex.execute(inv("kv-write", [pre + ".vc", pre + ".v"], pre + ".vc", {"row_offset": Integer(p)}))
        ex.execute(inv("attention", [pre + ".qr", pre + ".kc", pre + ".vc"], pre + ".out",
                       {"head_count": Integer(heads), "head_dimension": Integer(dim),
                        "kv_head_count": Integer(kv_heads), "causal": True,
                        "key_count": Integer(p + 1)}))
        if read:
            return ex.read_tensor(pre + ".out"), ex.read_tensor(pre + ".kc"), ex.read_tensor(pre + ".vc")

    def inputs(i):
        ex.write_tensor(pre + ".q", q_in[i])
        ex.write_tensor(pre + ".k", k_in[i])
        ex.write_tensor(pre + ".v", v_in[i])

    # The oracle's steps, on a host copy of the cache.
    kc_host, vc_host = history_k.copy(), history_v.copy()
    want = []
    for i, t in enumerate(offsets):
        p = start + t
        qr, _ = orc.rope(q_in[i], orc.rope_params(dim, heads, position_offset=p))
        kr, _ = orc.rope(k_in[i], orc.rope_params(dim, kv_heads, position_offset=p))
        kc_host[p] = kr[0]
        vc_host[p] = v_in[i][0]
        ap = orc.attention_params(1, capacity, heads, dim, kv_head_count=kv_heads, causal=True,
                                  key_count=p + 1)
        out, st = orc.attention(qr, kc_host, vc_host, ap)
        assert st == 0
        want.append((out, kr[0].copy()))

    # Eager steps at the same positions, in the same order.
    stores()
    eager = []
    for i, t in enumerate(offsets):
        inputs(i)
        eager.append(step(start + t))

    # Fresh stores; one eager step creates the outputs, then capture at p = start.
    stores()
    inputs(0)
    step(start)
    ex.begin_step_capture(["position_offset", "row_offset", "key_count"])
    step(start, read=False)
    capture = ex.end_step_capture()
    for i, t in enumerate(offsets):
        if i:
            ex.replay_step(capture, t, {pre + ".q": q_in[i], pre + ".k": k_in[i], pre + ".v": v_in[i]})
        out, kc, vc = (ex.read_tensor(pre + s) for s in (".out", ".kc", ".vc"))
        assert np.array_equal(bits(out), bits(eager[i][0])), t
        assert np.array_equal(bits(kc), bits(eager[i][1])), t
        assert np.array_equal(bits(vc), bits(eager[i][2])), t
        err = max_normwise_err(out, want[i][0])
        assert err <= 1e-4, (t, err)
        assert _rope_pair_err(kc[start + t], want[i][1]) <= 1e-6, t
        assert np.array_equal(bits(vc[start + t]), bits(v_in[i][0])), t
    ex.release_step_capture(capture)


def test_a_replay_keeps_a_flag_an_earlier_call_set(dev, orc):
    """A replay sets failure flags as eager calls do and clears none: an invalid
    embedding id recorded before a replay is still reported by the next check,
    and the check clears it."""
    import magnetar_hip
    from magnetar_hip import ops
    x = dev.upload(orc.normal(256, 5).reshape(1, 256))
    out = dev.empty((1, 256))
    ops.silu(dev, x, out=out)
    dev.capture_begin(0)
    ops.silu(dev, x, out=out)
    graph = dev.capture_end()
    table = dev.upload(orc.normal(32, 6).reshape(8, 4))
    ops.embedding(dev, table, dev.upload(np.array([9.0], np.float32)))  # id past the vocab
    graph.launch(0)
    with pytest.raises(magnetar_hip.MagnetarHipError):
        dev.check_flags()
    graph.launch(0)
    assert dev.check_flags() == 0
    want, _ = orc.silu(orc.normal(256, 5).reshape(1, 256))
    assert max_rel_err(out.numpy(), want) <= 1e-6
    graph.close()


BLOCK_CASES = [
    # hidden, heads, kv_heads, head_dim, ffn, cache rows, position, replay offsets
    (512, 8, 2, 64, 1024, 48, 20, (0, 1, 2, 3, 4)),
    # 16 query heads per KV head, captured past 256 keys, replayed far past them.
    (1024, 16, 1, 64, 1536, 420, 300, (0, 1, 57, 119)),
]


@pytest.mark.parametrize("hidden,heads,kv_heads,head_dim,ffn,rows,P,offsets", BLOCK_CASES)
def test_a_captured_decoder_block_replays_decode_steps(dev, orc, hidden, heads, kv_heads,
                                                       head_dim, ffn, rows, P, offsets):
    """mhip_block_forward captured once at position P (all three attributes
    advancing) and replayed at offset t equals the eager block at P + t bit
    for bit, and the oracle's block at P + t within the block's 1e-4."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from magnetar_hip.device import (ADVANCE_KEY_COUNT, ADVANCE_POSITION_OFFSET,
                                     ADVANCE_ROW_OFFSET)
    from reference_chain import reference_block
    s = Shapes(vocab=512, hidden=hidden, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=ffn)
    w = {}
    for i, (name, shape) in enumerate(s.weight_shapes().items()):
        n = int(np.prod(shape))
        w[name] = (orc.normal(n, 700 + i, 1.0, 0.1) if name.endswith("norm")
                   else orc.normal(n, 700 + i, 0.0, 0.02)).reshape(shape)
    kw = kv_heads * head_dim
    history_k = orc.normal(rows * kw, 790, 0.0, 0.5).reshape(rows, kw)
    history_v = orc.normal(rows * kw, 791, 0.0, 0.5).reshape(rows, kw)
    ids = [orc.token_ids(1, 800 + t, 512) for t in offsets]

    eager_block = DecoderBlock(dev, s, w, cache_rows=rows, max_seq=1)
    eager_block.k_cache, eager_block.v_cache = dev.upload(history_k), dev.upload(history_v)
    eager = []
    for i, t in enumerate(offsets):
        out = eager_block.forward(dev.upload(ids[i]), P + t).numpy()
        eager.append((out, eager_block.k_cache.numpy(), eager_block.v_cache.numpy()))

    kc_host, vc_host = history_k.copy(), history_v.copy()
    want = []
    for i, t in enumerate(offsets):
        out, kc_host, vc_host = reference_block(orc, s, w, ids[i], P + t, kc_host, vc_host)
        want.append(out)

    block = DecoderBlock(dev, s, w, cache_rows=rows, max_seq=1)
    block.k_cache, block.v_cache = dev.upload(history_k), dev.upload(history_v)
    ids_buf = dev.upload(ids[0])
    out = dev.empty((1, s.hidden))
    block.forward(ids_buf, P, out)  # sizes scratch and caches the RoPE table
    dev.capture_begin(ADVANCE_POSITION_OFFSET | ADVANCE_KEY_COUNT | ADVANCE_ROW_OFFSET)
    block.forward(ids_buf, P, out)
    graph = dev.capture_end()
    assert graph.max_offset == rows - (P + 1)
    for i, t in enumerate(offsets):
        dev.write(ids_buf, ids[i])
        graph.launch(t)
        got = out.numpy()
        assert np.array_equal(bits(got), bits(eager[i][0])), t
        assert np.array_equal(bits(block.k_cache.numpy()), bits(eager[i][1])), t
        assert np.array_equal(bits(block.v_cache.numpy()), bits(eager[i][2])), t
        err = max_normwise_err(got, want[i])
        assert err <= 1e-4, (t, err)
    import magnetar_hip
    with pytest.raises(magnetar_hip.MagnetarHipError):
        graph.launch(rows - P)  # past the cache
    dev.check_flags()
    graph.close()


def test_a_captured_decoder_block_replays_a_prefill_chunk(dev, orc):
    """A 16-token chunk of the block (its Q/K/V and gate/up sets and the O and
    down products on the one-launch small MFMA tiles, RoPE and the K/V cache
    append in the set's epilogue) captured at position P replays with new
    tokens: each replay equals the eager block at P bit for bit, and the
    oracle's block within 1e-4. Several query rows replay only at offset 0
    (src/kernels.rs:6661-6667), so the graph refuses any other."""
    import magnetar_hip
    from magnetar_hip import ops
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from magnetar_hip.device import (ADVANCE_KEY_COUNT, ADVANCE_POSITION_OFFSET,
                                     ADVANCE_ROW_OFFSET)
    from reference_chain import reference_block
    s = Shapes(vocab=512, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512)
    assert ops.matmul_plan(dev, 16, 256, 512)["path"] == "small_tiles"
    seq, rows, P = 16, 64, 8
    w = {}
    for i, (name, shape) in enumerate(s.weight_shapes().items()):
        n = int(np.prod(shape))
        w[name] = (orc.normal(n, 900 + i, 1.0, 0.1) if name.endswith("norm")
                   else orc.normal(n, 900 + i, 0.0, 0.05)).reshape(shape)
    kw = s.kv_heads * s.head_dim
    history_k = orc.normal(rows * kw, 990, 0.0, 0.5).reshape(rows, kw)
    history_v = orc.normal(rows * kw, 991, 0.0, 0.5).reshape(rows, kw)
    ids = [orc.token_ids(seq, 1000 + i, 512) for i in range(3)]

    eager_block = DecoderBlock(dev, s, w, cache_rows=rows, max_seq=seq)
    eager = []
    for i in range(3):
        eager_block.k_cache, eager_block.v_cache = dev.upload(history_k), dev.upload(history_v)
        out = eager_block.forward(dev.upload(ids[i]), P).numpy()
        eager.append((out, eager_block.k_cache.numpy(), eager_block.v_cache.numpy()))
        want, _, _ = reference_block(orc, s, w, ids[i], P, history_k.copy(), history_v.copy())
        assert max_normwise_err(out, want) <= 1e-4

    block = DecoderBlock(dev, s, w, cache_rows=rows, max_seq=seq)
    block.k_cache, block.v_cache = dev.upload(history_k), dev.upload(history_v)
    ids_buf = dev.upload(ids[0])
    out = dev.empty((seq, s.hidden))
    block.forward(ids_buf, P, out)  # sizes scratch and caches the RoPE table
    dev.capture_begin(ADVANCE_POSITION_OFFSET | ADVANCE_KEY_COUNT | ADVANCE_ROW_OFFSET)
    block.forward(ids_buf, P, out)
    graph = dev.capture_end()
    assert graph.max_offset == 0
    for i in (1, 0, 2, 1):
        dev.write(ids_buf, ids[i])
        graph.launch(0)
        assert np.array_equal(bits(out.numpy()), bits(eager[i][0])), i
        assert np.array_equal(bits(block.k_cache.numpy()), bits(eager[i][1])), i
        assert np.array_equal(bits(block.v_cache.numpy()), bits(eager[i][2])), i
    with pytest.raises(magnetar_hip.MagnetarHipError):
        graph.launch(1)
    dev.check_flags()
    graph.close()


def test_queued_replays_each_keep_their_own_offset(dev, orc):
    """A RoPE step (position advancing) and a kv-write step (row advancing),
    replayed at 64 offsets back to back with no wait between replays: each
    replay's launches copy their arguments when issued, so every replay
    writes its own row at its own position, bit for bit the eager RoPE
    there. The offsets cover the offset table's first size, its growth (5000,
    100000) and, past its reach (2^22 + 123), the word written ahead of the
    launches."""
    from magnetar_hip import ops
    from magnetar_hip.device import ADVANCE_POSITION_OFFSET, ADVANCE_ROW_OFFSET
    width, P, capacity = 256, 3, 4096
    x = orc.normal(width, 91).reshape(1, width)
    dx = dev.upload(x)
    offsets = list(range(56)) + [4095, 4000, 5000, 100000, 17, (1 << 22) + 123, 2, 99999]
    eager = {t: ops.rope(dev, dx, ops.rope_params(64, 4, position_offset=P + t)).numpy()
             for t in set(offsets)}
    for t in (0, 100000, (1 << 22) + 123):
        want, st = orc.rope(x, orc.rope_params(64, 4, position_offset=P + t))
        assert st == 0 and max_normwise_err(eager[t], want) <= 1e-6
    y = dev.empty((1, width))
    store = dev.zeros((P + capacity + 1, width))
    dev.sync()
    dev.capture_begin(ADVANCE_POSITION_OFFSET)
    ops.rope(dev, dx, ops.rope_params(64, 4, position_offset=P), out=y)
    step_rope = dev.capture_end()
    dev.capture_begin(ADVANCE_ROW_OFFSET)
    ops.kv_write(dev, store, y, P)
    step_row = dev.capture_end()
    assert step_rope.max_offset >= (1 << 22) + 123
    assert step_row.max_offset == capacity
    want_rows = {}
    for t in offsets:
        step_rope.launch(t)
        step_row.launch(t % capacity)  # queued behind the RoPE replay, no wait
        want_rows[P + t % capacity] = eager[t]  # a later replay of a row wins
    got = store.numpy()
    for row, want in want_rows.items():
        assert np.array_equal(bits(got[row]), bits(want[0])), row
    untouched = sorted(set(range(P + capacity + 1)) - set(want_rows))
    assert not np.any(got[untouched])
    step_rope.close()
    step_row.close()
