"""numpy bindings of the CPU oracle (oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker or the timed CPU baseline; the product never does.
Every function returns (result, status) where status is the mhip_status value
the reference would fail with (0 when it succeeds).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_I = ctypes.c_int


class RopeParams(ctypes.Structure):
    _fields_ = [
        ("base", ctypes.c_float),
        ("scale", ctypes.c_float),
        ("dimension", ctypes.c_uint64),
        ("position_offset", ctypes.c_uint64),
        ("head_count", ctypes.c_uint64),
        ("half_split", ctypes.c_uint32),
        ("rotated_pairs", ctypes.c_uint64),
        ("banded_factor", ctypes.c_float),
        ("low_freq_factor", ctypes.c_float),
        ("high_freq_factor", ctypes.c_float),
        ("original_context_length", ctypes.c_float),
        ("yarn_factor", ctypes.c_float),
        ("yarn_low", ctypes.c_float),
        ("yarn_high", ctypes.c_float),
        ("amplitude", ctypes.c_float),
    ]


class AttentionParams(ctypes.Structure):
    _fields_ = [
        ("seq_len", ctypes.c_uint64),
        ("kv_rows", ctypes.c_uint64),
        ("kv_seq_len", ctypes.c_uint64),
        ("head_count", ctypes.c_uint64),
        ("kv_head_count", ctypes.c_uint64),
        ("head_dimension", ctypes.c_uint64),
        ("value_dimension", ctypes.c_uint64),
        ("causal", ctypes.c_int),
        ("window_size", ctypes.c_int64),
        ("scale", ctypes.c_float),
    ]


_SIGS = {
    "orc_hashed_values": [_P, _U64, _U64],
    "orc_values": [_P, _U64, _U64],
    "orc_attention_values": [_P, _U64, _U64],
    "orc_uniform": [_P, _U64, _U64, _F, _F],
    "orc_normal": [_P, _U64, _U64, _F, _F],
    "orc_token_ids": [_P, _U64, _U64, _U64],
    "orc_f16_to_f32": [ctypes.c_uint16],
    "orc_bf16_to_f32": [ctypes.c_uint16],
    "orc_f32_to_f16": [_F],
    "orc_f32_to_bf16": [_F],
    "orc_encode_f16": [_P, _P, _U64],
    "orc_encode_bf16": [_P, _P, _U64],
    "orc_decode_f16": [_P, _P, _U64],
    "orc_decode_bf16": [_P, _P, _U64],
    "orc_half_binary": [_P, _P, _P, _U64, _I, _I],
    "orc_add": [_P, _P, _P, _U64],
    "orc_bias_add": [_P, _P, _P, _U64, _U64],
    "orc_mul": [_P, _P, _P, _U64],
    "orc_mul_scalar": [_P, _P, _P, _U64],
    "orc_silu": [_P, _P, _U64],
    "orc_silu_mul": [_P, _P, _P, _U64],
    "orc_scale": [_P, _P, _F, _U64],
    "orc_embedding": [_P, _U64, _U64, _P, _U64, _P],
    "orc_rmsnorm": [_P, _P, _P, _U64, _U64, _U64, _F],
    "orc_softmax_rows": [_P, _P, _U64, _U64],
    "orc_rope_frequencies": [ctypes.POINTER(RopeParams), _P, _P],
    "orc_rope": [_P, _P, _U64, _U64, ctypes.POINTER(RopeParams)],
    "orc_matmul": [_P, _P, _P, _U64, _U64, _U64, _I, _I, _P, _I],
    "orc_matmul_rows": [_P, _P, _P, _U64, _U64, _U64, _U64],
    "orc_attention": [_P, _P, _P, _P, ctypes.POINTER(AttentionParams)],
    "orc_attention_heads": [_P, _P, _P, _P, ctypes.POINTER(AttentionParams), _U64, _U64],
    "orc_greedy_select": [_P, _U64, _P, ctypes.c_uint32, _F],
}
_RES = {
    "orc_f16_to_f32": ctypes.c_float,
    "orc_bf16_to_f32": ctypes.c_float,
    "orc_f32_to_f16": ctypes.c_uint16,
    "orc_f32_to_bf16": ctypes.c_uint16,
    "orc_greedy_select": ctypes.c_int64,
}
_VOID = {"orc_hashed_values", "orc_values", "orc_attention_values", "orc_uniform", "orc_normal",
         "orc_token_ids", "orc_encode_f16", "orc_encode_bf16", "orc_decode_f16",
         "orc_decode_bf16", "orc_half_binary", "orc_add", "orc_mul", "orc_mul_scalar",
         "orc_silu", "orc_silu_mul", "orc_scale", "orc_rope_frequencies", "orc_matmul_rows"}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        handle = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = _RES.get(name, None if name in _VOID else ctypes.c_int)
        _lib = handle
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- generators ----
def hashed_values(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_hashed_values(_ptr(out), n, seed)
    return out


def values(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_values(_ptr(out), n, seed)
    return out


def attention_values(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_attention_values(_ptr(out), n, seed)
    return out


def uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_uniform(_ptr(out), n, seed, lo, hi)
    return out


def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_normal(_ptr(out), n, seed, mean, std)
    return out


def token_ids(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_token_ids(_ptr(out), n, seed, vocab)
    return out


# ---- half codec ----
def encode_half(x, dtype: int) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    (lib().orc_encode_bf16 if dtype else lib().orc_encode_f16)(_ptr(x), _ptr(out), x.size)
    return out


def decode_half(h, dtype: int) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    (lib().orc_decode_bf16 if dtype else lib().orc_decode_f16)(_ptr(h), _ptr(out), h.size)
    return out


def half_binary(a, b, dtype: int, op: str) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(a.shape, np.uint16)
    lib().orc_half_binary(_ptr(a), _ptr(b), _ptr(out), a.size, dtype, 1 if op == "mul" else 0)
    return out


# ---- f32 kernels ----
def add(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().orc_add(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out, 0


def bias_add(a, bias):
    a, bias = _f32(a), _f32(bias)
    out = np.empty_like(a)
    st = lib().orc_bias_add(_ptr(a), _ptr(bias), _ptr(out), bias.size, a.size)
    return out, st


def mul(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().orc_mul(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out, 0


def mul_scalar(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().orc_mul_scalar(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out, 0


def silu(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_silu(_ptr(x), _ptr(out), x.size)
    return out, 0


def silu_mul(g, u):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    lib().orc_silu_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out, 0


def scale(x, factor):
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_scale(_ptr(x), _ptr(out), factor, x.size)
    return out, 0


def embedding(table, ids):
    table, ids = _f32(table), _f32(ids)
    vocab, dim = table.shape
    out = np.zeros((ids.size, dim), np.float32)
    st = lib().orc_embedding(_ptr(table), vocab, dim, _ptr(ids), ids.size, _ptr(out))
    return out, st


def rmsnorm(x, weight, eps, cols=None, weight_row_stride=0):
    x = _f32(x)
    cols = cols if cols is not None else x.shape[-1]
    w = _f32(weight) if weight is not None else None
    out = np.empty_like(x)
    st = lib().orc_rmsnorm(_ptr(x), _ptr(w) if w is not None else None, _ptr(out),
                           x.size // cols, cols, weight_row_stride, eps)
    return out, st


def softmax_rows(x):
    x = _f32(x)
    rows, cols = x.shape
    out = np.zeros_like(x)
    st = lib().orc_softmax_rows(_ptr(x), _ptr(out), rows, cols)
    return out, st


def rope_params(dimension, head_count=1, **kw) -> RopeParams:
    p = RopeParams()
    p.base, p.scale, p.dimension, p.head_count = 10000.0, 1.0, dimension, head_count
    p.rotated_pairs, p.amplitude = dimension // 2, 1.0
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def rope_frequencies(params: RopeParams):
    half = params.dimension // 2
    freq = np.empty(half, np.float32)
    amp = np.empty(half, np.float32)
    lib().orc_rope_frequencies(ctypes.byref(params), _ptr(freq), _ptr(amp))
    return freq, amp


def rope(x, params: RopeParams):
    x = _f32(x)
    rows, cols = x.shape
    out = np.empty_like(x)
    st = lib().orc_rope(_ptr(x), _ptr(out), rows, cols, ctypes.byref(params))
    return out, st


def matmul(a, b, transpose_a=False, transpose_b=False, addend=None, addend_mode=0):
    a, b = _f32(a), _f32(b)
    m, k = (a.shape[1], a.shape[0]) if transpose_a else a.shape
    k2, n = (b.shape[1], b.shape[0]) if transpose_b else b.shape
    if k != k2:
        return None, 1
    out = np.empty((m, n), np.float32)
    ad = _f32(addend) if addend is not None else None
    st = lib().orc_matmul(_ptr(a), _ptr(b), _ptr(out), m, k, n, int(transpose_a),
                          int(transpose_b), _ptr(ad) if ad is not None else None, addend_mode)
    return out, st


def matmul_rows(a, b, row_begin, row_end):
    a, b = _f32(a), _f32(b)
    k = a.shape[1]
    n = b.shape[1]
    out = np.empty((row_end - row_begin, n), np.float32)
    lib().orc_matmul_rows(_ptr(a), _ptr(b), _ptr(out), row_begin, row_end, k, n)
    return out


def attention_params(seq_len, kv_rows, head_count, head_dimension, kv_head_count=None,
                     value_dimension=None, causal=False, window_size=None, key_count=None,
                     scale=None) -> AttentionParams:
    p = AttentionParams()
    p.seq_len, p.kv_rows = seq_len, kv_rows
    p.kv_seq_len = key_count if key_count is not None else kv_rows
    p.head_count = head_count
    p.kv_head_count = kv_head_count if kv_head_count is not None else head_count
    p.head_dimension = head_dimension
    p.value_dimension = value_dimension if value_dimension is not None else head_dimension
    p.causal = int(bool(causal))
    p.window_size = -1 if window_size is None else window_size
    p.scale = 0.0 if scale is None else scale
    return p


def attention(q, k, v, params: AttentionParams, heads=None):
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros((params.seq_len, params.head_count * params.value_dimension), np.float32)
    if heads is None:
        st = lib().orc_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), ctypes.byref(params))
    else:
        st = lib().orc_attention_heads(_ptr(q), _ptr(k), _ptr(v), _ptr(out),
                                       ctypes.byref(params), heads[0], heads[1])
    return out, st


def greedy_select(row, excluded=(), temperature=0.0):
    """Column index or None (orc_greedy_select)."""
    row = _f32(row).ravel()
    flat = np.array([v for r in excluded for v in (r[0], r[1])] or [0, 0], np.uint64)
    col = lib().orc_greedy_select(_ptr(row), row.size, _ptr(flat), len(excluded),
                                  ctypes.c_float(temperature))
    return None if col < 0 else int(col)
