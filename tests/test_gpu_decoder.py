"""GPU: the decoder-block chain (BASELINE configs 0 and 4) against the same
chain on the CPU oracle, including decode steps through the in-place KV cache.

Bar: 1e-4 normwise relative error on the block output (the chain composes
matmul / rmsnorm / attention, each held to 1e-4, and the elementwise ops)."""
import numpy as np
import pytest

from conftest import max_normwise_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


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
    from magnetar_hip.decoder import DecoderBlock, Shapes, reference_block
    s = Shapes(vocab=1024, hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=688)
    w = weights_for(orc, s, 100)
    block = DecoderBlock(dev, s, w, cache_rows=64, max_seq=32)
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
    from magnetar_hip.decoder import DecoderBlock, Shapes, reference_block
    s = Shapes(vocab=512, hidden=512, heads=8, kv_heads=2, head_dim=64, ffn=1024, eps=1e-6,
               rope_base=500000.0)
    w = weights_for(orc, s, 200)
    block = DecoderBlock(dev, s, w, cache_rows=80, max_seq=70)
    ids = orc.token_ids(70, 8, 512)
    got = block.forward(dev.upload(ids), 0).numpy()
    want, _, _ = reference_block(orc, s, w, ids, 0, np.zeros((80, 128), np.float32),
                                 np.zeros((80, 128), np.float32))
    assert max_normwise_err(got, want) <= TOL


def test_llama2_7b_block_decode_at_kv_2048(dev, orc):
    """Config 4 decode: hidden 4096, 32 x 128 heads, FFN 11008, one token at
    position 2048 against 2048 cached K/V rows."""
    from magnetar_hip.decoder import DecoderBlock, Shapes, reference_block
    s = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    w = weights_for(orc, s, 300)
    rows = 2049
    block = DecoderBlock(dev, s, w, cache_rows=rows, max_seq=1)
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
    print(f"llama2-7b decode: {err:.2e}")
    assert err <= TOL


def test_llama2_7b_block_prefill(dev, orc):
    """Config 4 prefill shape at 64 tokens (the oracle's CPU time bounds the length)."""
    from magnetar_hip.decoder import DecoderBlock, Shapes, reference_block
    s = Shapes(vocab=32000, hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    w = weights_for(orc, s, 400)
    block = DecoderBlock(dev, s, w, cache_rows=64, max_seq=64)
    ids = orc.token_ids(64, 401, 32000)
    got = block.forward(dev.upload(ids), 0).numpy()
    want, _, _ = reference_block(orc, s, w, ids, 0, np.zeros((64, 4096), np.float32),
                                 np.zeros((64, 4096), np.float32))
    err = max_normwise_err(got, want)
    print(f"llama2-7b prefill(64): {err:.2e}")
    assert err <= TOL
