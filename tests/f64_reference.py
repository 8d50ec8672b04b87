"""Float64 statements of the hot-path kernels and the decoder-block chain --
TEST INFRASTRUCTURE: the "exact" anchor that both the device's results and the
CPU oracle's are measured against, so that an elementwise error can be
attributed to a kernel or to f32 summation order.

Each function is the textbook mathematics of the reference's kernel
(src/kernels.cu:1098-1138 rmsnorm, :1232-1260 softmax, :1147-1229 rope,
:1262-1306 matmul, :1868-1959 attention, :64-79 silu) evaluated in f64 from the
same f32 inputs. Two steps stay f32 because the reference defines them in f32
and both implementations compute them identically: a RoPE angle is the f32
product `(float)position * frequency` of the f32 frequency table
(src/kernels.cu:1197-1221), and the embedding gather is a copy.
"""
from __future__ import annotations

import numpy as np


def f64(x) -> np.ndarray:
    return np.asarray(x, np.float64)


def matmul(a, b, addend=None) -> np.ndarray:
    out = f64(a) @ f64(b)
    if addend is not None:
        out = out + f64(addend)
    return out


def abs_product(a, b) -> np.ndarray:
    """|A| |B| in f64: the scale of the gamma_k forward-error bound."""
    return np.abs(f64(a)) @ np.abs(f64(b))


def gamma(k: int) -> float:
    """gamma_k = k u / (1 - k u), u = 2^-24: any order of f32 multiply-adds over
    k terms errs by at most gamma_k (|A||B|)_ij (Higham, Accuracy and Stability
    of Numerical Algorithms, 2nd ed., eq. 3.5)."""
    u = 2.0 ** -24
    return k * u / (1.0 - k * u)


def rmsnorm(x, w, eps) -> np.ndarray:
    x = f64(x)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + float(eps))
    return x * inv * (f64(w) if w is not None else 1.0)


def softmax_rows(x) -> np.ndarray:
    x = f64(x)
    e = np.exp(x - np.max(x, axis=-1, keepdims=True))
    return e / np.sum(e, axis=-1, keepdims=True)


def silu(x) -> np.ndarray:
    x = f64(x)
    return x / (1.0 + np.exp(-x))


def rope(orc, x, params) -> np.ndarray:
    """Interleaved or half-split rotation of every head of x (f32 or f64
    values), with the reference's f32 angles and f64 sin, cos and products."""
    x = f64(x)
    rows, cols = x.shape
    H, dim = int(params.head_count), int(params.dimension)
    half, width = dim // 2, cols // H
    freq, amp = orc.rope_frequencies(params)
    pos = (np.arange(rows, dtype=np.uint64) + np.uint64(params.position_offset)).astype(np.float32) \
        * np.float32(params.scale)
    angle = (pos[:, None] * np.asarray(freq, np.float32)[None, :]).astype(np.float64)  # f32 product
    s, c = np.sin(angle) * f64(amp)[None, :], np.cos(angle) * f64(amp)[None, :]
    out = x.copy()
    for h in range(H):
        base = h * width
        if params.half_split:
            i0 = base + np.arange(half)
            i1 = i0 + half
        else:
            i0 = base + 2 * np.arange(half)
            i1 = i0 + 1
        a, b = x[:, i0], x[:, i1]
        out[:, i0] = a * c - b * s
        out[:, i1] = a * s + b * c
    return out


def attention(q, k, v, seq, H, Hkv, d, vd=None, causal=True, key_count=None, window=None,
              scale=None, heads=None) -> np.ndarray:
    """softmax(q k^T * scale + mask) v per head, f64; query i sits at position
    (key_count - seq) + i; `heads` limits the computed heads (others stay 0)."""
    vd = vd or d
    q, k, v = f64(q), f64(k), f64(v)
    kv = key_count if key_count is not None else k.shape[0]
    sc = scale if scale else 1.0 / np.sqrt(np.float32(d))  # 1/sqrtf(d), as the reference's f32
    sc = float(np.float32(sc))
    out = np.zeros((seq, H * vd))
    group = H // Hkv
    qpos = (kv - seq) + np.arange(seq)
    keys = np.arange(kv)
    mask = np.ones((seq, kv), bool)
    if causal:
        mask &= keys[None, :] <= qpos[:, None]
        if window is not None and window > 0:
            mask &= keys[None, :] >= (qpos[:, None] - (window - 1))
    for h in range(H) if heads is None else range(*heads):
        g = h // group
        s = q[:, h * d:(h + 1) * d] @ k[:kv, g * d:(g + 1) * d].T * sc
        s = np.where(mask, s, -np.inf)
        m = np.max(s, axis=1, keepdims=True)
        ok = np.isfinite(m[:, 0])
        p = np.where(mask, np.exp(s - np.where(np.isfinite(m), m, 0.0)), 0.0)
        p = p / np.where(ok[:, None], p.sum(axis=1, keepdims=True), 1.0)
        out[:, h * vd:(h + 1) * vd] = p @ v[:kv, g * vd:(g + 1) * vd]
    return out


def block(orc, shapes, weights: dict, ids, position: int, k_cache, v_cache):
    """The decoder-block chain of tests/reference_chain.reference_block in f64:
    (out, k_cache, v_cache), the caches as f64 copies with the new rows."""
    s = shapes
    table = np.asarray(weights["embedding"], np.float32)
    x = f64(table[np.asarray(ids).astype(np.int64)])
    h = rmsnorm(x, weights["attn_norm"], s.eps)
    q = h @ f64(weights["wq"])
    k = h @ f64(weights["wk"])
    v = h @ f64(weights["wv"])
    q = rope(orc, q, orc.rope_params(s.head_dim, s.heads, base=s.rope_base, position_offset=position))
    k = rope(orc, k, orc.rope_params(s.head_dim, s.kv_heads, base=s.rope_base,
                                     position_offset=position))
    seq = len(ids)
    kc, vc = f64(k_cache).copy(), f64(v_cache).copy()
    kc[position:position + seq] = k
    vc[position:position + seq] = v
    a = attention(q, kc, vc, seq, s.heads, s.kv_heads, s.head_dim, causal=True,
                  key_count=position + seq)
    x2 = a @ f64(weights["wo"]) + x
    h2 = rmsnorm(x2, weights["ffn_norm"], s.eps)
    f = silu(h2 @ f64(weights["w_gate"])) * (h2 @ f64(weights["w_up"]))
    return f @ f64(weights["w_down"]) + x2, kc, vc


def rel_err_significant(actual, exact, frac: float = 1e-3) -> float:
    """max |a - e| / |e| over entries with |e| >= frac * max |e| (the
    elementwise relative error where it is defined)."""
    a = f64(actual).reshape(-1)
    e = f64(exact).reshape(-1)
    if a.size == 0:
        return 0.0
    keep = np.abs(e) >= frac * float(np.max(np.abs(e)))
    return float(np.max(np.abs(a[keep] - e[keep]) / np.abs(e[keep]))) if keep.any() else 0.0
