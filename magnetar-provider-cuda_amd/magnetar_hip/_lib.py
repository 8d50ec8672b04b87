"""ctypes declarations for libmagnetar_hip.so (include/magnetar_hip.h).

The library is built in-tree by ``make -C magnetar-provider-cuda_amd`` (or
``__graft_entry__.build()``). Importing this module without the built library
raises ImportError: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmagnetar_hip.so")

STATUS_NAMES = {
    0: "Ok",
    1: "ShapeUnsupported",
    2: "DTypeUnsupported",
    3: "LayoutUnsupported",
    4: "ExecutionFailed",
    5: "OutOfDeviceMemory",
    6: "CompilationFailed",
    7: "DriverFailed",
    8: "DeviceUnavailable",
    9: "CaptureUnsupported",
}

MHIP_F16 = 0
MHIP_BF16 = 1
FLAG_EMBEDDING_INVALID_ID = 1
FLAG_SOFTMAX_NON_FINITE = 2


class MagnetarHipError(RuntimeError):
    """A non-Ok ``mhip_status`` with the library's redacted detail string."""

    def __init__(self, status: int, detail: str):
        self.status = status
        self.code = STATUS_NAMES.get(status, f"Unknown({status})")
        self.detail = detail
        super().__init__(f"{self.code}: {detail}")


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("ordinal", ctypes.c_int),
        ("name", ctypes.c_char * 256),
        ("architecture", ctypes.c_char * 64),
        ("total_memory", ctypes.c_uint64),
        ("free_memory", ctypes.c_uint64),
        ("compute_units", ctypes.c_uint32),
        ("wavefront_size", ctypes.c_uint32),
        ("lds_per_workgroup", ctypes.c_uint64),
        ("pressure", ctypes.c_int),
    ]


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


class MatmulPlan(ctypes.Structure):
    """mhip_matmul_plan: the kernel path mhip_matmul_f32 takes for a shape."""
    _fields_ = [("path", ctypes.c_uint32), ("tile_m", ctypes.c_uint32), ("tile_n", ctypes.c_uint32),
                ("waves", ctypes.c_uint32), ("splits", ctypes.c_uint32), ("stream_k", ctypes.c_uint32)]


MATMUL_PATHS = {0: "gemv", 1: "gemv_row_blocks", 2: "tiles", 3: "small_tiles"}


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
        ("batch", ctypes.c_uint64),
        ("q_batch_stride", ctypes.c_uint64),
        ("kv_batch_stride", ctypes.c_uint64),
        ("v_batch_stride", ctypes.c_uint64),
        ("out_batch_stride", ctypes.c_uint64),
        ("bounded_key_count", ctypes.c_uint32),
    ]


_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_I = ctypes.c_int
_CTX = ctypes.c_void_p

# name -> argtypes (every function returns mhip_status as int unless listed in _RESTYPES)
SIGNATURES = {
    "mhip_last_error_detail": [],
    "mhip_status_name": [_I],
    "mhip_version": [],
    "mhip_device_count": [ctypes.POINTER(_I)],
    "mhip_ctx_create": [_I, ctypes.POINTER(_CTX)],
    "mhip_ctx_destroy": [_CTX],
    "mhip_device_query": [_CTX, ctypes.POINTER(DeviceInfo)],
    "mhip_alloc": [_CTX, ctypes.c_size_t, ctypes.POINTER(_P)],
    "mhip_free": [_CTX, _P],
    "mhip_upload": [_CTX, _P, _P, ctypes.c_size_t],
    "mhip_download": [_CTX, _P, _P, ctypes.c_size_t],
    "mhip_copy": [_CTX, _P, _P, ctypes.c_size_t],
    "mhip_zero": [_CTX, _P, ctypes.c_size_t],
    "mhip_sync": [_CTX],
    "mhip_check_flags": [_CTX, ctypes.POINTER(ctypes.c_uint32)],
    "mhip_timer_start": [_CTX],
    "mhip_timer_stop": [_CTX, ctypes.POINTER(_F)],
    "mhip_add_f32": [_CTX, _P, _P, _P, _U64],
    "mhip_bias_add_f32": [_CTX, _P, _P, _P, _U64, _U64],
    "mhip_mul_f32": [_CTX, _P, _P, _P, _U64],
    "mhip_mul_scalar_f32": [_CTX, _P, _P, _P, _U64],
    "mhip_silu_f32": [_CTX, _P, _P, _U64],
    "mhip_silu_mul_f32": [_CTX, _P, _P, _P, _U64],
    "mhip_scale_f32": [_CTX, _P, _P, _F, _U64],
    "mhip_add_half": [_CTX, _P, _P, _P, _U64, _I],
    "mhip_mul_half": [_CTX, _P, _P, _P, _U64, _I],
    "mhip_encode_half": [_CTX, _P, _P, _U64, _I],
    "mhip_decode_half": [_CTX, _P, _P, _U64, _I],
    "mhip_embedding_f32": [_CTX, _P, _U64, _U64, _P, _U64, _P],
    "mhip_rmsnorm_f32": [_CTX, _P, _P, _P, _U64, _U64, _U64, _F],
    "mhip_softmax_rows_f32": [_CTX, _P, _P, _U64, _U64],
    "mhip_rope_params_default": [ctypes.POINTER(RopeParams), _U64, _U64],
    "mhip_rope_f32": [_CTX, _P, _P, _U64, _U64, ctypes.POINTER(RopeParams)],
    "mhip_matmul_f32": [_CTX, _P, _P, _P, _U64, _U64, _U64, _I, _I, _P, _I],
    "mhip_matmul_f32_noalloc": [_CTX, _P, _P, _P, _U64, _U64, _U64, _I, _I, _P, _I],
    "mhip_matmul_plan_f32": [_CTX, _U64, _U64, _U64, _I, _I, ctypes.POINTER(MatmulPlan)],
    "mhip_attention_f32": [_CTX, _P, _P, _P, _P, ctypes.POINTER(AttentionParams)],
    "mhip_kv_write_f32": [_CTX, _P, _U64, _U64, _P, _U64, _U64],
    "mhip_matmul_bf16w_f32": [_CTX, _P, _P, _P, _U64, _U64, _U64, ctypes.c_int, ctypes.c_int, _P,
                              ctypes.c_int],
    "mhip_embedding_bf16w_f32": [_CTX, _P, _U64, _U64, _P, _U64, _P],
    "mhip_greedy_select_f32": [_CTX, _P, _U64, _U64, _U64, _P, ctypes.c_uint32, ctypes.c_float,
                               ctypes.POINTER(ctypes.c_int64)],
    "mhip_capture_begin": [_CTX, ctypes.c_uint32],
    "mhip_capture_end": [_CTX, ctypes.POINTER(_P), ctypes.POINTER(_U64)],
    "mhip_capture_abort": [_CTX],
    "mhip_graph_launch": [_P, _U64],
    "mhip_graph_destroy": [_P],
    "mhip_capture_active": [_CTX],
    "mhip_graph_max_offset": [_P],
}

_RESTYPES = {
    "mhip_last_error_detail": ctypes.c_char_p,
    "mhip_status_name": ctypes.c_char_p,
    "mhip_version": ctypes.c_char_p,
    "mhip_rope_params_default": None,
    "mhip_graph_max_offset": _U64,
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads the library once; raises ImportError if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C magnetar-provider-cuda_amd` "
                "or __graft_entry__.build(); there is no non-HIP fallback"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = handle
    return _lib


def check(status: int) -> None:
    """Raises MagnetarHipError for a non-Ok status."""
    if status != 0:
        detail = lib().mhip_last_error_detail()
        raise MagnetarHipError(status, detail.decode() if detail else "")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
