"""A Llama-style decoder block on the device (mhip_block_forward), with its
weights, KV cache and workspace held as DeviceArrays."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .device import Device, DeviceArray


class BlockConfig(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_uint64), ("heads", ctypes.c_uint64),
                ("kv_heads", ctypes.c_uint64), ("head_dim", ctypes.c_uint64),
                ("ffn", ctypes.c_uint64), ("vocab", ctypes.c_uint64),
                ("eps", ctypes.c_float), ("rope_base", ctypes.c_float),
                ("weight_format", ctypes.c_uint32)]


class BlockWeights(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("embedding", "attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up",
                 "w_down")]


WEIGHT_NAMES = ("embedding", "attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up",
                "w_down")

SIGNATURES = ("mhip_block_workspace_bytes", "mhip_block_forward")
_bound = False


def _bind():
    global _bound
    lib = _lib.lib()
    if not _bound:
        lib.mhip_block_workspace_bytes.argtypes = [ctypes.POINTER(BlockConfig), ctypes.c_uint64]
        lib.mhip_block_workspace_bytes.restype = ctypes.c_uint64
        lib.mhip_block_forward.argtypes = [ctypes.c_void_p, ctypes.POINTER(BlockConfig),
                                           ctypes.POINTER(BlockWeights), ctypes.c_void_p,
                                           ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                           ctypes.c_uint64, ctypes.c_void_p]
        lib.mhip_block_forward.restype = ctypes.c_int
        _bound = True
    return lib


@dataclass
class Shapes:
    vocab: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    eps: float = 1e-5
    rope_base: float = 10000.0

    def weight_shapes(self):
        H, Hk, d, h, f = self.heads, self.kv_heads, self.head_dim, self.hidden, self.ffn
        return {"embedding": (self.vocab, h), "attn_norm": (h,), "wq": (h, H * d),
                "wk": (h, Hk * d), "wv": (h, Hk * d), "wo": (H * d, h), "ffn_norm": (h,),
                "w_gate": (h, f), "w_up": (h, f), "w_down": (f, h)}


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """The bf16 bit patterns of f32 values that are exactly bf16 values."""
    u = np.ascontiguousarray(values, np.float32).view(np.uint32)
    if np.any(u & 0xFFFF):
        raise ValueError("values are not exact bf16 values")
    return (u >> 16).astype(np.uint16)


class DecoderBlock:
    def __init__(self, dev: Device, shapes: Shapes, weights: dict, cache_rows: int,
                 max_seq: int, bf16_weights: bool = False):
        """`bf16_weights`: store the matrices compact, as bf16 bit patterns (host
        values must be exact bf16 values; device arrays must hold the bits)."""
        self.dev, self.s, self.cache_rows = dev, shapes, cache_rows

        def place(name, v):
            if isinstance(v, DeviceArray):
                return v
            v = np.asarray(v, np.float32)
            if bf16_weights and not name.endswith("norm"):
                return dev.upload(bf16_bits(v))
            return dev.upload(v)

        self.w = {k: place(k, v) for k, v in weights.items()}
        kv = shapes.kv_heads * shapes.head_dim
        self.k_cache = dev.zeros((cache_rows, kv))
        self.v_cache = dev.zeros((cache_rows, kv))
        self.cfg = BlockConfig(shapes.hidden, shapes.heads, shapes.kv_heads, shapes.head_dim,
                               shapes.ffn, shapes.vocab, shapes.eps, shapes.rope_base,
                               1 if bf16_weights else 0)
        self.cw = BlockWeights(*[self.w[n].ptr for n in WEIGHT_NAMES])
        self.ws_bytes = int(_bind().mhip_block_workspace_bytes(ctypes.byref(self.cfg), max_seq))
        self.ws = dev.empty((max(1, self.ws_bytes // 4),))
        self.max_seq = max_seq

    def forward(self, ids: DeviceArray, position: int, out: DeviceArray | None = None) -> DeviceArray:
        seq = ids.size
        if seq > self.max_seq:
            raise ValueError("more tokens than the workspace was sized for")
        out = out if out is not None else self.dev.empty((seq, self.s.hidden))
        _lib.check(_bind().mhip_block_forward(
            self.dev.ctx, ctypes.byref(self.cfg), ctypes.byref(self.cw), ctypes.c_void_p(ids.ptr),
            seq, position, ctypes.c_void_p(self.k_cache.ptr), ctypes.c_void_p(self.v_cache.ptr),
            self.cache_rows, ctypes.c_void_p(self.ws.ptr), self.ws_bytes, ctypes.c_void_p(out.ptr)))
        return out

