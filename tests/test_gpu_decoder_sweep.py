"""GPU parity: seeded random decoder-block shapes. Each case draws the widths
(heads, grouping, head size, FFN), the number of rows and the cache position
from its seed; the fused block must equal the same chain as separate ABI calls
bit for bit (output and cache rows) and the CPU oracle's block within 1e-4
normwise."""
import numpy as np
import pytest

from conftest import max_normwise_err, sweep_seeds
from test_gpu_decoder import poisoned, unfused_block, weights_for

pytestmark = pytest.mark.gpu


def draw(seed):
    rng = np.random.default_rng(60_000 + seed)
    head_dim = int(rng.choice([32, 64, 128]))
    heads = int(rng.choice([2, 4, 8]))
    kv_heads = int(rng.choice([h for h in (1, 2, 4, 8) if heads % h == 0]))
    ffn = 4 * int(rng.integers(32, 400))
    vocab = int(rng.integers(256, 2048))
    seq = int(rng.choice([1, 2, 5, 8, 16, 24, 32, int(rng.integers(1, 48))]))
    position = int(rng.integers(0, 40))
    return head_dim, heads, kv_heads, ffn, vocab, seq, position


@pytest.mark.parametrize("seed", sweep_seeds(16))
def test_random_block(dev, orc, seed):
    from magnetar_hip.decoder import DecoderBlock, Shapes
    from reference_chain import reference_block
    head_dim, heads, kv_heads, ffn, vocab, seq, position = draw(seed)
    hidden = heads * head_dim
    s = Shapes(vocab=vocab, hidden=hidden, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
               ffn=ffn)
    w = weights_for(orc, s, 900 + 20 * seed)
    for i, name in enumerate(("attn_norm", "ffn_norm")):  # gains other than 1
        w[name] = 1.0 + 0.1 * orc.normal(hidden, 940 + 2 * seed + i, 0.0, 1.0)
    rows = position + seq + 3
    kv_dim = kv_heads * head_dim
    block = poisoned(DecoderBlock(dev, s, w, cache_rows=rows, max_seq=seq))
    kc = orc.normal(rows * kv_dim, 910 + seed, 0.0, 0.5).reshape(rows, kv_dim)
    vc = orc.normal(rows * kv_dim, 920 + seed, 0.0, 0.5).reshape(rows, kv_dim)
    block.k_cache = dev.upload(kc)
    block.v_cache = dev.upload(vc)
    k2, v2 = dev.upload(kc), dev.upload(vc)
    ids_host = orc.token_ids(seq, 930 + seed, vocab)
    ids = dev.upload(ids_host)
    got = block.forward(ids, position).numpy()
    sep = unfused_block(dev, s, block.w, ids, position, k2, v2).numpy()
    dev.check_flags()
    print(f"seed {seed}: hidden {hidden} heads {heads}/{kv_heads}x{head_dim} ffn {ffn} "
          f"seq {seq} at {position}")
    assert np.array_equal(got.view(np.uint32), sep.view(np.uint32))
    assert np.array_equal(block.k_cache.numpy().view(np.uint32), k2.numpy().view(np.uint32))
    want, _, _ = reference_block(orc, s, w, ids_host, position, kc.copy(), vc.copy())
    err = max_normwise_err(got, want)
    print(f"  vs oracle: {err:.2e}")
    assert err <= 1e-4
