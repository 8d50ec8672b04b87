"""The decoder-block chain on the CPU oracle: the checker for the device's
mhip_block_forward (tests, smoke() and the bench's CPU baseline).

The chain is the reference's hardware hot-path block
(src/tests_hardware_hot_path.rs:339-526): embedding gather, rmsnorm, Q/K/V
projections, RoPE on Q and K at the block's position, the new K/V rows written
into the cache at that position, causal attention over key_count = position +
seq, output projection + residual, rmsnorm, SwiGLU (silu(gate) * up), down
projection + residual.

Large products are split by rows (and attention by heads) over host threads.
Each output element is still one orc_matmul_rows / orc_attention_heads sum, in
the oracle's order, so the values are those of the single-threaded oracle
calls (ctypes releases the GIL during each call).
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np


def host_threads() -> int:
    """Threads for the oracle: this process's CPUs, at most 16 (a GPU box's share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _spans(total: int, parts: int):
    parts = max(1, min(parts, total))
    step = (total + parts - 1) // parts
    return [(i, min(total, i + step)) for i in range(0, total, step)]


def matmul(orc, a, b, addend=None, threads: int | None = None):
    """a[m,k] @ b[k,n] (+ addend[m,n] after the sum, as orc_matmul's residual
    mode), rows split over threads; equal to orc.matmul bit for bit."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m = a.shape[0]
    if threads is None:
        small = m * a.shape[1] * b.shape[1] < (1 << 24)
        threads = 1 if small else host_threads()
    if threads == 1:
        out, st = orc.matmul(a, b, addend=addend, addend_mode=2 if addend is not None else 0)
        assert st == 0
        return out
    with ThreadPoolExecutor(threads) as pool:
        parts = list(pool.map(lambda s: orc.matmul_rows(a, b, s[0], s[1]), _spans(m, threads)))
    out = np.concatenate(parts, axis=0)
    if addend is not None:
        out = out + np.asarray(addend, np.float32)  # one f32 rounding, as o + addend
    return out


def attention(orc, q, k, v, params, threads: int | None = None):
    """orc.attention with the heads split over threads (each head is computed
    by itself in the oracle, so the split changes no value)."""
    threads = threads or host_threads()
    H, vd = params.head_count, params.value_dimension
    if threads == 1 or H == 1:
        out, st = orc.attention(q, k, v, params)
        assert st == 0
        return out
    out = np.zeros((params.seq_len, H * vd), np.float32)

    def run(span):
        part, st = orc.attention(q, k, v, params, heads=span)
        assert st == 0
        return span, part

    with ThreadPoolExecutor(threads) as pool:
        for (h0, h1), part in pool.map(run, _spans(H, threads)):
            out[:, h0 * vd:h1 * vd] = part[:, h0 * vd:h1 * vd]
    return out


def reference_block(orc, shapes, weights: dict, ids, position: int, k_cache, v_cache,
                    threads: int | None = None):
    """The block on the oracle; returns (out, k_cache, v_cache) with the new
    K/V rows written at `position` (copies; the arguments are not changed)."""
    s = shapes
    x, st = orc.embedding(weights["embedding"], ids)
    assert st == 0
    h, _ = orc.rmsnorm(x, weights["attn_norm"], s.eps)
    q = matmul(orc, h, weights["wq"], threads=threads)
    k = matmul(orc, h, weights["wk"], threads=threads)
    v = matmul(orc, h, weights["wv"], threads=threads)
    q, _ = orc.rope(q, orc.rope_params(s.head_dim, s.heads, base=s.rope_base, position_offset=position))
    k, _ = orc.rope(k, orc.rope_params(s.head_dim, s.kv_heads, base=s.rope_base, position_offset=position))
    seq = len(ids)
    k_cache = k_cache.copy()
    v_cache = v_cache.copy()
    k_cache[position:position + seq] = k
    v_cache[position:position + seq] = v
    p = orc.attention_params(seq, k_cache.shape[0], s.heads, s.head_dim, kv_head_count=s.kv_heads,
                             causal=True, key_count=position + seq)
    a = attention(orc, q, k_cache, v_cache, p, threads=threads)
    x2 = matmul(orc, a, weights["wo"], addend=x, threads=threads)
    h2, _ = orc.rmsnorm(x2, weights["ffn_norm"], s.eps)
    g = matmul(orc, h2, weights["w_gate"], threads=threads)
    u = matmul(orc, h2, weights["w_up"], threads=threads)
    f, _ = orc.silu_mul(g, u)
    out = matmul(orc, f, weights["w_down"], addend=x2, threads=threads)
    return out, k_cache, v_cache
