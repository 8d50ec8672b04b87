"""Magnetar MI355X Provider: Python bindings over libmagnetar_hip.so.

The product is the C ABI in include/magnetar_hip.h (HIP kernels for gfx950
plus the C++ executor); this package only binds it for tests, the benchmark
and Python callers. Importing it requires the built library.
"""
from ._lib import MagnetarHipError, STATUS_NAMES, MHIP_F16, MHIP_BF16, lib  # noqa: F401
from .device import Device, DeviceArray, device_count  # noqa: F401
from . import ops  # noqa: F401
from .executor import (Provider, Executor, KernelInvocation, TensorRef, KernelError,  # noqa: F401
                       Float, Integer, Boolean, String, DType, F32, F16, BF16)

lib()  # fail loudly at import when the library is missing

__version__ = "0.1.0"
