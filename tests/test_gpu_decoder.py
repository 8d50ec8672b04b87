"""GPU: the decoder-block chain (BASELINE configs 0 and 4) against the same
chain on the CPU oracle, including decode steps through the in-place KV cache.

Bar: 1e-4 normwise relative error on the block output (the chain composes
matmul / rmsnorm / attention, each held to 1e-4, and the elementwise ops)."""
import numpy as np
import pytest

from conftest import max_normwise_err, max_rel_err_significant

pytestmark = pytest.mark.gpu

TOL = 1e-4


def poisoned(block):
    """The block with NaN in every workspace float, so a value read before the
    block writes it shows up in the output rather than depending on what the
    allocation held before."""
    import ctypes
    from magnetar_hip._lib import call
    nan = np.full(block.ws.shape, np.nan, np.float32)
    call("mhip_upload", block.dev.ctx, ctypes.c_void_p(block.ws.ptr), nan.ctypes.data_as(ctypes.c_void_p),
         nan.nbytes)
    return block


def weights_for(orc, shapes, seed=0):
    w = {}
    for i, (name, shape) in enumerate(shapes.weight_shapes().items()):
        n = int(np.prod(shape))
        if name.endswith("norm"):
            w[name] = np.ones(shape, np.float32)  # gain = 1
        else:
            w[name] = orc.normal(n, seed + i, 0.0, 0.02).reshape(shape)
    return w


def test_tiny_block_prefill_and_decode(dev, orc):
    """Config 0: vocab 1024, hidden 256, 4 heads x 64, seq 32, FFN 688; then
    four decode steps appending to the cache."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from reference_chain import reference_block
    s = Shapes(vocab=1024, hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=688)
    w = weights_for(orc, s, 100)
    block = poisoned(DecoderBlock(dev, s, w, cache_rows=64, max_seq=32))
    ids = orc.token_ids(32, 7, 1024)
    got = block.forward(dev.upload(ids), 0).numpy()
    dev.check_flags()
    kc = np.zeros((64, 256), np.float32)
    vc = np.zeros((64, 256), np.float32)
    want, kc, vc = reference_block(orc, s, w, ids, 0, kc, vc)
    assert max_normwise_err(got, want) <= TOL
    assert max_normwise_err(block.k_cache.numpy()[:32], kc[:32]) <= TOL
    for step in range(4):
        tok = orc.token_ids(1, 50 + step, 1024)
        got = block.forward(dev.upload(tok), 32 + step).numpy()
        want, kc, vc = reference_block(orc, s, w, tok, 32 + step, kc, vc)
        err = max_normwise_err(got, want)
        print(f"decode step {step}: {err:.2e}")
        assert err <= TOL


def test_gqa_block(dev, orc):
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from reference_chain import reference_block
    s = Shapes(vocab=512, hidden=512, heads=8, kv_heads=2, head_dim=64, ffn=1024, eps=1e-6,
               rope_base=500000.0)
    w = weights_for(orc, s, 200)
    block = poisoned(DecoderBlock(dev, s, w, cache_rows=80, max_seq=70))
    ids = orc.token_ids(70, 8, 512)
    got = block.forward(dev.upload(ids), 0).numpy()
    want, _, _ = reference_block(orc, s, w, ids, 0, np.zeros((80, 128), np.float32),
                                 np.zeros((80, 128), np.float32))
    assert max_normwise_err(got, want) <= TOL


def test_decode_over_more_than_256_key_chunks(dev, orc):
    """One token against a 33,000-row cache: the attention leaves 258 key
    chunks per head, more than the merge's 256 threads take in one stride,
    and the O projection's launch merges them (its k slices of 32 lie inside
    64-wide heads). Bit-identical to the separate calls, within 1e-4 of the
    oracle's block."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from reference_chain import reference_block
    s = Shapes(vocab=256, hidden=128, heads=2, kv_heads=2, head_dim=64, ffn=256)
    w = weights_for(orc, s, 700)
    for i, name in enumerate(("attn_norm", "ffn_norm")):
        w[name] = 1.0 + 0.1 * orc.normal(128, 710 + i, 0.0, 1.0)
    position = 33000
    rows = position + 1
    kc = np.zeros((rows, 128), np.float32)
    vc = np.zeros((rows, 128), np.float32)
    kc[:position] = orc.normal(position * 128, 701, 0.0, 0.5).reshape(position, 128)
    vc[:position] = orc.normal(position * 128, 702, 0.0, 0.5).reshape(position, 128)
    block = poisoned(DecoderBlock(dev, s, w, cache_rows=rows, max_seq=1))
    block.k_cache = dev.upload(kc)
    block.v_cache = dev.upload(vc)
    k2, v2 = dev.upload(kc), dev.upload(vc)
    tok = orc.token_ids(1, 703, 256)
    ids = dev.upload(tok)
    got = block.forward(ids, position).numpy()
    sep = unfused_block(dev, s, block.w, ids, position, k2, v2).numpy()
    dev.check_flags()
    assert np.array_equal(got.view(np.uint32), sep.view(np.uint32))
    want, _, _ = reference_block(orc, s, w, tok, position, kc, vc)
    assert max_normwise_err(got, want) <= TOL


def test_llama2_7b_block_decode_at_kv_2048(dev, orc):
    """Config 4 decode: hidden 4096, 32 x 128 heads, FFN 11008, one token at
    position 2048 against 2048 cached K/V rows."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from reference_chain import reference_block
    s = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    w = weights_for(orc, s, 300)
    rows = 2049
    block = poisoned(DecoderBlock(dev, s, w, cache_rows=rows, max_seq=1))
    kc = np.zeros((rows, 4096), np.float32)
    vc = np.zeros((rows, 4096), np.float32)
    kc[:2048] = orc.normal(2048 * 4096, 301, 0.0, 0.5).reshape(2048, 4096)
    vc[:2048] = orc.normal(2048 * 4096, 302, 0.0, 0.5).reshape(2048, 4096)
    block.k_cache = dev.upload(kc)
    block.v_cache = dev.upload(vc)
    tok = orc.token_ids(1, 303, 32000)
    got = block.forward(dev.upload(tok), 2048).numpy()
    want, _, _ = reference_block(orc, s, w, tok, 2048, kc, vc)
    err = max_normwise_err(got, want)
    print(f"llama2-7b decode: {err:.2e}, elementwise (|ref| >= 1e-3 max) "
          f"{max_rel_err_significant(got, want):.2e}")
    assert err <= TOL


def test_llama2_7b_block_prefill(dev, orc):
    """Config 4 prefill: the BASELINE's 512 tokens at position 0 (hidden 4096,
    32 x 128 heads, FFN 11008), output and the K/V rows the block writes."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from reference_chain import reference_block
    s = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    w = weights_for(orc, s, 400)
    seq = 512
    block = DecoderBlock(dev, s, w, cache_rows=seq, max_seq=seq)
    ids = orc.token_ids(seq, 401, 32000)
    got = block.forward(dev.upload(ids), 0).numpy()
    want, kc, vc = reference_block(orc, s, w, ids, 0, np.zeros((seq, 4096), np.float32),
                                   np.zeros((seq, 4096), np.float32))
    err = max_normwise_err(got, want)
    k_err = max_normwise_err(block.k_cache.numpy(), kc)
    v_err = max_normwise_err(block.v_cache.numpy(), vc)
    print(f"llama2-7b prefill(512): out {err:.2e}, K rows {k_err:.2e}, V rows {v_err:.2e}, "
          f"elementwise out (|ref| >= 1e-3 max) {max_rel_err_significant(got, want):.2e}")
    assert err <= TOL and k_err <= TOL and v_err <= TOL


def _rows_view(arr, first, count):
    """Rows [first, first + count) of a 2-D device array, without a copy."""
    from magnetar_hip.device import DeviceArray
    cols = arr.shape[1]
    return DeviceArray(arr.device, arr.ptr + first * cols * 4, (count, cols), arr.dtype,
                       arr.half, owned=False)


def unfused_block(dev, s, w, ids, position, k_cache, v_cache):
    """The block as separate ABI calls (embedding, rmsnorm, three matmuls, two
    RoPEs, attention, matmul-residual, rmsnorm, two matmuls, silu-mul,
    matmul-residual), writing new K/V rows into the given caches."""
    from magnetar_hip import ops
    seq = ids.size
    x = ops.embedding(dev, w["embedding"], ids)
    h = ops.rmsnorm(dev, x, w["attn_norm"], s.eps)
    q = ops.matmul(dev, h, w["wq"])
    k_rows = _rows_view(k_cache, position, seq)
    v_rows = _rows_view(v_cache, position, seq)
    ops.matmul(dev, h, w["wk"], out=k_rows)
    ops.matmul(dev, h, w["wv"], out=v_rows)
    ops.rope(dev, q, ops.rope_params(s.head_dim, s.heads, base=s.rope_base,
                                     position_offset=position), out=q)
    ops.rope(dev, k_rows, ops.rope_params(s.head_dim, s.kv_heads, base=s.rope_base,
                                          position_offset=position), out=k_rows)
    p = ops.attention_params(seq, k_cache.shape[0], s.heads, s.head_dim, kv_head_count=s.kv_heads,
                             causal=True, key_count=position + seq)
    a = ops.attention(dev, q, k_cache, v_cache, p)
    x2 = ops.matmul(dev, a, w["wo"], addend=x, addend_mode=2)
    h2 = ops.rmsnorm(dev, x2, w["ffn_norm"], s.eps)
    g = ops.matmul(dev, h2, w["w_gate"])
    u = ops.matmul(dev, h2, w["w_up"])
    f = ops.silu_mul(dev, g, u)
    return ops.matmul(dev, f, w["w_down"], addend=x2, addend_mode=2)


@pytest.mark.parametrize("seq,position,hidden", [(1, 40, 512), (3, 20, 512), (8, 0, 512), (16, 8, 512),
                                                 (24, 0, 512), (32, 0, 512), (20, 4, 512), (40, 0, 512),
                                                 (1, 40, 256), (1, 7, 2048), (1, 0, 4096),
                                                 (4, 3, 2048), (8, 0, 4096), (16, 5, 2048)])
def test_fused_block_is_bit_identical_to_the_separate_calls(dev, orc, seq, position, hidden):
    """The decode fusions (embedding + rmsnorm; for one token the attention
    merge inside the O projection's launch and the FFN RMSNorm inside the
    gate/up launch; Q/K/V GEMVs with RoPE in the reduction, gate/up GEMVs with
    silu * up) change launches, not arithmetic: the block output and the
    cache rows equal the unfused chain's bit for bit. 16-32 rows take the sets
    on one-launch MFMA tiles where k <= 1024 (Q/K/V, O, gate/up here) and in
    row blocks of 8 on the GEMV otherwise (the down projection's k = 1376);
    20 and 40 rows take the separate calls in the block too. Hidden 256/512 normalise a row with one wave, 2048/4096 with a
    workgroup of four."""
    from magnetar_hip.decoder import DecoderBlock, Shapes
    head_dim = 64 if hidden <= 512 else 128
    s = Shapes(vocab=1024, hidden=hidden, heads=hidden // head_dim, kv_heads=2, head_dim=head_dim,
               ffn=1376)
    w = weights_for(orc, s, 500)
    for name in ("attn_norm", "ffn_norm"):  # gains other than 1, so their order shows
        w[name] = 1.0 + 0.1 * orc.normal(hidden, 510 + len(name), 0.0, 1.0)
    rows = 64
    block = poisoned(DecoderBlock(dev, s, w, cache_rows=rows, max_seq=40))
    kv = s.kv_heads * s.head_dim
    kc = orc.normal(rows * kv, 501, 0.0, 0.5).reshape(rows, kv)
    vc = orc.normal(rows * kv, 502, 0.0, 0.5).reshape(rows, kv)
    block.k_cache = dev.upload(kc)
    block.v_cache = dev.upload(vc)
    k2, v2 = dev.upload(kc), dev.upload(vc)
    ids = dev.upload(orc.token_ids(seq, 503 + seq, 1024))
    got = block.forward(ids, position).numpy()
    want = unfused_block(dev, s, block.w, ids, position, k2, v2).numpy()
    dev.check_flags()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(block.k_cache.numpy().view(np.uint32), k2.numpy().view(np.uint32))
    assert np.array_equal(block.v_cache.numpy().view(np.uint32), v2.numpy().view(np.uint32))


def test_decode_block_rejects_an_invalid_token_id(dev, orc):
    """The fused embedding + rmsnorm raises the embedding's invalid-id flag."""
    import magnetar_hip
    from magnetar_hip.decoder import DecoderBlock, Shapes
    s = Shapes(vocab=64, hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=512)
    block = DecoderBlock(dev, s, weights_for(orc, s, 600), cache_rows=8, max_seq=2)
    block.forward(dev.upload(np.array([3.0], np.float32)), 0)
    dev.check_flags()
    block.forward(dev.upload(np.array([64.0], np.float32)), 1)
    with pytest.raises(magnetar_hip.MagnetarHipError):
        dev.check_flags()
