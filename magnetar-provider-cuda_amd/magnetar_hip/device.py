"""A bound MI355X device and its device-resident arrays (numpy in, numpy out).

This is the Python view of the C ABI's context and buffer entry points; it
owns nothing but the handles. Shapes and dtypes ride along with each buffer
the way `CudaDeviceBuffer` carries its shape (reference src/kernels.rs:253-379).
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import MagnetarHipError, call, lib


def device_count() -> int:
    n = ctypes.c_int(0)
    call("mhip_device_count", ctypes.byref(n))
    return n.value


class DeviceArray:
    """A device allocation with a shape and a numpy dtype (f32, or uint16 for halves)."""

    __slots__ = ("device", "ptr", "shape", "dtype", "nbytes", "half", "_owned", "__weakref__")

    def __init__(self, device: "Device", ptr: int, shape: Sequence[int], dtype, half=None,
                 owned: bool = True):
        self.device = device
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.half = half  # None for f32, else _lib.MHIP_F16 / MHIP_BF16
        self._owned = owned

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def free(self) -> None:
        if self._owned and self.ptr:
            lib().mhip_free(self.device.ctx, ctypes.c_void_p(self.ptr))
        self.ptr = 0
        self._owned = False

    def __del__(self):
        try:
            if self._owned and self.ptr and self.device.ctx:
                lib().mhip_free(self.device.ctx, ctypes.c_void_p(self.ptr))
        except Exception:
            pass

    def numpy(self) -> np.ndarray:
        return self.device.download(self)

    def __repr__(self):
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, half={self.half})"


class Device:
    """One HIP device context (`mhip_ctx`): a single in-order stream."""

    def __init__(self, ordinal: int = 0):
        handle = ctypes.c_void_p()
        call("mhip_ctx_create", ordinal, ctypes.byref(handle))
        self.ctx = handle
        self.ordinal = ordinal

    def close(self) -> None:
        if self.ctx:
            lib().mhip_ctx_destroy(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        info = _lib.DeviceInfo()
        call("mhip_device_query", self.ctx, ctypes.byref(info))
        return {
            "ordinal": info.ordinal,
            "name": info.name.decode(),
            "architecture": info.architecture.decode(),
            "total_memory": info.total_memory,
            "free_memory": info.free_memory,
            "compute_units": info.compute_units,
            "wavefront_size": info.wavefront_size,
            "lds_per_workgroup": info.lds_per_workgroup,
            "pressure": info.pressure,
        }

    # ---- buffers ----
    def empty(self, shape: Sequence[int], dtype=np.float32, half=None) -> DeviceArray:
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        ptr = ctypes.c_void_p()
        call("mhip_alloc", self.ctx, nbytes, ctypes.byref(ptr))
        return DeviceArray(self, ptr.value or 0, shape, dtype, half)

    def zeros(self, shape: Sequence[int], dtype=np.float32, half=None) -> DeviceArray:
        arr = self.empty(shape, dtype, half)
        call("mhip_zero", self.ctx, ctypes.c_void_p(arr.ptr), arr.nbytes)
        return arr

    def upload(self, host: np.ndarray, half=None) -> DeviceArray:
        host = np.ascontiguousarray(host)
        arr = self.empty(host.shape, host.dtype, half)
        if arr.nbytes:
            call("mhip_upload", self.ctx, ctypes.c_void_p(arr.ptr),
                 host.ctypes.data_as(ctypes.c_void_p), arr.nbytes)
        return arr

    def write(self, arr: DeviceArray, host: np.ndarray) -> DeviceArray:
        """Copies `host` into the existing buffer `arr` (same byte size)."""
        host = np.ascontiguousarray(host, dtype=arr.dtype)
        if host.nbytes != arr.nbytes:
            raise ValueError(f"write of {host.nbytes} bytes into a {arr.nbytes}-byte buffer")
        if arr.nbytes:
            call("mhip_upload", self.ctx, ctypes.c_void_p(arr.ptr),
                 host.ctypes.data_as(ctypes.c_void_p), arr.nbytes)
        return arr

    def download(self, arr: DeviceArray) -> np.ndarray:
        out = np.empty(arr.shape, dtype=arr.dtype)
        call("mhip_download", self.ctx, out.ctypes.data_as(ctypes.c_void_p),
             ctypes.c_void_p(arr.ptr), arr.nbytes)
        return out

    def sync(self) -> None:
        call("mhip_sync", self.ctx)

    def check_flags(self) -> int:
        flags = ctypes.c_uint32(0)
        call("mhip_check_flags", self.ctx, ctypes.byref(flags))
        return flags.value

    def timer_start(self) -> None:
        call("mhip_timer_start", self.ctx)

    def timer_stop(self) -> float:
        ms = ctypes.c_float(0.0)
        call("mhip_timer_stop", self.ctx, ctypes.byref(ms))
        return ms.value


    # ---- step capture (mhip_capture_*) ----
    def capture_begin(self, advancing: int = 0) -> None:
        """Records the following launches into a graph instead of running them;
        `advancing` is a mask of ADVANCE_* attributes a replay offset moves."""
        call("mhip_capture_begin", self.ctx, advancing)

    def capture_end(self) -> "CapturedStep":
        handle = ctypes.c_void_p()
        bound = ctypes.c_uint64(0)
        call("mhip_capture_end", self.ctx, ctypes.byref(handle), ctypes.byref(bound))
        return CapturedStep(self, handle, bound.value)

    def capture_abort(self) -> None:
        call("mhip_capture_abort", self.ctx)


ADVANCE_POSITION_OFFSET, ADVANCE_KEY_COUNT, ADVANCE_ROW_OFFSET = 1, 2, 4


class CapturedStep:
    """A captured launch sequence; launch(offset) re-issues it on the stream with
    every advancing attribute increased by `offset` (at most `max_offset`)."""

    def __init__(self, device: Device, handle, max_offset: int):
        self.device, self._h, self.max_offset = device, handle, max_offset

    def launch(self, offset: int = 0) -> None:
        call("mhip_graph_launch", self._h, offset)

    def close(self) -> None:
        # A closed device took its graphs' memory with it.
        if self._h and self.device.ctx:
            lib().mhip_graph_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["Device", "DeviceArray", "CapturedStep", "MagnetarHipError", "device_count",
           "ADVANCE_POSITION_OFFSET", "ADVANCE_KEY_COUNT", "ADVANCE_ROW_OFFSET"]
