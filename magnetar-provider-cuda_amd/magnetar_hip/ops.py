"""Thin calls of the C ABI's kernel entry points on DeviceArrays.

Each function enqueues one launch on the device's stream and returns the
output array; nothing waits unless the caller downloads or checks flags.
Sizes come from the arrays; shape rules beyond element counts belong to the
executor (the reference's `CudaKernels` layer).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import call
from .device import Device, DeviceArray


def _p(arr: DeviceArray | None):
    return ctypes.c_void_p(arr.ptr if arr is not None else 0)


def _out(dev: Device, out, shape, dtype=np.float32, half=None):
    return out if out is not None else dev.empty(shape, dtype, half)


def add(dev: Device, a: DeviceArray, b: DeviceArray, out=None) -> DeviceArray:
    out = _out(dev, out, a.shape)
    call("mhip_add_f32", dev.ctx, _p(a), _p(b), _p(out), a.size)
    return out


def bias_add(dev: Device, a: DeviceArray, bias: DeviceArray, out=None) -> DeviceArray:
    out = _out(dev, out, a.shape)
    call("mhip_bias_add_f32", dev.ctx, _p(a), _p(bias), _p(out), bias.size, a.size)
    return out


def mul(dev: Device, a: DeviceArray, b: DeviceArray, out=None) -> DeviceArray:
    out = _out(dev, out, a.shape)
    call("mhip_mul_f32", dev.ctx, _p(a), _p(b), _p(out), a.size)
    return out


def mul_scalar(dev: Device, a: DeviceArray, b: DeviceArray, out=None) -> DeviceArray:
    out = _out(dev, out, a.shape)
    call("mhip_mul_scalar_f32", dev.ctx, _p(a), _p(b), _p(out), a.size)
    return out


def silu(dev: Device, x: DeviceArray, out=None) -> DeviceArray:
    out = _out(dev, out, x.shape)
    call("mhip_silu_f32", dev.ctx, _p(x), _p(out), x.size)
    return out


def silu_mul(dev: Device, gate: DeviceArray, up: DeviceArray, out=None) -> DeviceArray:
    out = _out(dev, out, gate.shape)
    call("mhip_silu_mul_f32", dev.ctx, _p(gate), _p(up), _p(out), gate.size)
    return out


def scale(dev: Device, x: DeviceArray, factor: float, out=None) -> DeviceArray:
    out = _out(dev, out, x.shape)
    call("mhip_scale_f32", dev.ctx, _p(x), _p(out), ctypes.c_float(factor), x.size)
    return out


def half_binary(dev: Device, a: DeviceArray, b: DeviceArray, op: str, dtype: int,
                out=None) -> DeviceArray:
    out = _out(dev, out, a.shape, np.uint16, dtype)
    name = "mhip_add_half" if op == "add" else "mhip_mul_half"
    call(name, dev.ctx, _p(a), _p(b), _p(out), a.size, dtype)
    return out


def encode_half(dev: Device, x: DeviceArray, dtype: int, out=None) -> DeviceArray:
    out = _out(dev, out, x.shape, np.uint16, dtype)
    call("mhip_encode_half", dev.ctx, _p(x), _p(out), x.size, dtype)
    return out


def decode_half(dev: Device, x: DeviceArray, dtype: int, out=None) -> DeviceArray:
    out = _out(dev, out, x.shape)
    call("mhip_decode_half", dev.ctx, _p(x), _p(out), x.size, dtype)
    return out


def embedding(dev: Device, table: DeviceArray, ids: DeviceArray, out=None) -> DeviceArray:
    vocab, dim = table.shape
    out = _out(dev, out, (ids.size, dim))
    call("mhip_embedding_f32", dev.ctx, _p(table), vocab, dim, _p(ids), ids.size, _p(out))
    return out


def rmsnorm(dev: Device, x: DeviceArray, weight: DeviceArray | None, eps: float,
            cols: int | None = None, weight_row_stride: int = 0, out=None) -> DeviceArray:
    cols = cols if cols is not None else x.shape[-1]
    rows = x.size // cols
    out = _out(dev, out, x.shape)
    call("mhip_rmsnorm_f32", dev.ctx, _p(x), _p(weight), _p(out), rows, cols,
         weight_row_stride, ctypes.c_float(eps))
    return out


def softmax_rows(dev: Device, x: DeviceArray, out=None) -> DeviceArray:
    rows, cols = x.shape
    out = _out(dev, out, x.shape)
    call("mhip_softmax_rows_f32", dev.ctx, _p(x), _p(out), rows, cols)
    return out


def rope_params(dimension: int, head_count: int = 1, **kw) -> _lib.RopeParams:
    p = _lib.RopeParams()
    _lib.lib().mhip_rope_params_default(ctypes.byref(p), dimension, head_count)
    for key, value in kw.items():
        setattr(p, key, value)
    return p


def rope(dev: Device, x: DeviceArray, params: _lib.RopeParams, out=None) -> DeviceArray:
    rows, cols = x.shape
    out = _out(dev, out, x.shape)
    call("mhip_rope_f32", dev.ctx, _p(x), _p(out), rows, cols, ctypes.byref(params))
    return out


def matmul(dev: Device, a: DeviceArray, b: DeviceArray, transpose_a: bool = False,
           transpose_b: bool = False, addend: DeviceArray | None = None, addend_mode: int = 0,
           out=None) -> DeviceArray:
    m, k = (a.shape[1], a.shape[0]) if transpose_a else (a.shape[0], a.shape[1])
    k2, n = (b.shape[1], b.shape[0]) if transpose_b else (b.shape[0], b.shape[1])
    if k != k2:
        raise ValueError(f"matmul inner dimension mismatch: {k} vs {k2}")
    out = _out(dev, out, (m, n))
    call("mhip_matmul_f32", dev.ctx, _p(a), _p(b), _p(out), m, k, n, int(transpose_a),
         int(transpose_b), _p(addend), addend_mode)
    return out


def matmul_plan(dev: Device, m: int, k: int, n: int, transpose_a: bool = False,
                transpose_b: bool = False) -> dict:
    """The kernel path mhip_matmul_f32 takes for an m x k x n product with
    aligned operands: {"path": "gemv" | "gemv_row_blocks" | "tiles", "tile":
    (tile_m, tile_n), "waves", "splits", "stream_k"}."""
    p = _lib.MatmulPlan()
    call("mhip_matmul_plan_f32", dev.ctx, m, k, n, int(transpose_a), int(transpose_b),
         ctypes.byref(p))
    return {"path": _lib.MATMUL_PATHS[p.path], "tile": (p.tile_m, p.tile_n), "waves": p.waves,
            "splits": p.splits, "stream_k": bool(p.stream_k)}


def attention_params(seq_len, kv_rows, head_count, head_dimension, kv_head_count=None,
                     value_dimension=None, causal=False, window_size=None, key_count=None,
                     scale=None, batch=1) -> _lib.AttentionParams:
    p = _lib.AttentionParams()
    p.seq_len, p.kv_rows = seq_len, kv_rows
    p.kv_seq_len = key_count if key_count is not None else kv_rows
    p.head_count = head_count
    p.kv_head_count = kv_head_count if kv_head_count is not None else head_count
    p.head_dimension = head_dimension
    p.value_dimension = value_dimension if value_dimension is not None else head_dimension
    p.causal = int(bool(causal))
    p.window_size = -1 if window_size is None else window_size
    p.scale = 0.0 if scale is None else scale
    p.batch = batch
    p.bounded_key_count = int(key_count is not None)
    return p


def attention(dev: Device, q: DeviceArray, k: DeviceArray, v: DeviceArray,
              params: _lib.AttentionParams, out=None) -> DeviceArray:
    batch = max(1, params.batch)
    rows = params.seq_len * batch
    out = _out(dev, out, (rows, params.head_count * params.value_dimension))
    call("mhip_attention_f32", dev.ctx, _p(q), _p(k), _p(v), _p(out), ctypes.byref(params))
    return out


def kv_write(dev: Device, store: DeviceArray, rows: DeviceArray, row_offset: int) -> DeviceArray:
    """store[row_offset : row_offset + len(rows)] = rows, in place (kv-write)."""
    capacity, width = store.shape
    count = rows.shape[0] if rows.shape else 0
    if rows.size != count * width:
        raise ValueError("kv-write rows must be [count, store width]")
    call("mhip_kv_write_f32", dev.ctx, _p(store), capacity, width, _p(rows), count, row_offset)
    return store


def greedy_select(dev: Device, logits: DeviceArray, row: int = 0, excluded=(),
                  temperature: float = 0.0):
    """Greedy column of `logits` row `row`, or None (mhip_greedy_select_f32)."""
    cols = logits.shape[-1]
    rows = logits.size // max(1, cols)
    flat = [int(v) for r in excluded for v in (r[0], r[1])]
    ranges = (ctypes.c_uint64 * max(1, len(flat)))(*flat)
    col = ctypes.c_int64(-1)
    call("mhip_greedy_select_f32", dev.ctx, _p(logits), rows, cols, row, ranges, len(flat) // 2,
         temperature, ctypes.byref(col))
    return None if col.value < 0 else int(col.value)


def matmul_bf16w(dev: Device, a: DeviceArray, b_bits: DeviceArray, transpose_a: bool = False,
                 transpose_b: bool = False, addend: DeviceArray | None = None,
                 addend_mode: int = 0, out=None) -> DeviceArray:
    """matmul with a compact weight: b as bf16 bit patterns (uint16)."""
    m, k = (a.shape[1], a.shape[0]) if transpose_a else (a.shape[0], a.shape[1])
    k2, n = (b_bits.shape[1], b_bits.shape[0]) if transpose_b else (b_bits.shape[0], b_bits.shape[1])
    if k != k2:
        raise ValueError(f"matmul inner dimension mismatch: {k} vs {k2}")
    out = _out(dev, out, (m, n))
    call("mhip_matmul_bf16w_f32", dev.ctx, _p(a), _p(b_bits), _p(out), m, k, n, int(transpose_a),
         int(transpose_b), _p(addend), addend_mode)
    return out


def embedding_bf16w(dev: Device, table_bits: DeviceArray, ids: DeviceArray, out=None) -> DeviceArray:
    vocab, dim = table_bits.shape
    out = _out(dev, out, (ids.size, dim))
    call("mhip_embedding_bf16w_f32", dev.ctx, _p(table_bits), vocab, dim, _p(ids), ids.size, _p(out))
    return out
