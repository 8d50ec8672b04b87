"""Python view of the Provider / Executor C ABI (include/magnetar_hip.h).

Names follow the reference's Rust API so tests read like its own:
`Provider.health()`, `.devices()`, `.kernel_advertisements()`,
`.execution_api()`; `Executor.write_tensor`, `.read_tensor`, `.submit_kernel`,
`.complete_kernel` (reference src/provider.rs:250-324, src/executor.rs:2244-2565).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import _lib

F32, F16, BF16 = 0, 1, 2
# KV store precisions (KvStorePrecision); only KV_F32 stores are provided.
KV_F32, KV_TQ4, KV_TQ3 = 0, 1, 2
DTYPE_NAMES = {F32: "Float32", F16: "Float16", BF16: "BrainFloat16"}

KERNEL_ERRORS = {
    0: "Ok",
    1: "KernelShapeUnsupported",
    2: "KernelDTypeUnsupported",
    3: "KernelLayoutUnsupported",
    4: "KernelDeviceUnsupported",
    5: "KernelOutOfDeviceMemory",
    6: "KernelExecutionFailed",
    7: "KernelAttributeUnsupported",
    8: "KernelNotFound",
    9: "KernelTimeout",
    10: "StepReplayInvalidated",
}
HEALTH = {0: "Available", 1: "Degraded", 2: "Unavailable"}
OBSERVATIONS = {0: "KernelDispatchStarted", 1: "KernelDispatchCompleted",
                2: "KernelDispatchFailed", 3: "KernelTimeout"}


class KernelError(RuntimeError):
    def __init__(self, code: int, detail: str):
        self.code = KERNEL_ERRORS.get(code, f"Unknown({code})")
        self.detail = detail
        super().__init__(f"{self.code}: {detail}")


# ---- C structures ----
class _Attribute(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("kind", ctypes.c_int), ("f", ctypes.c_double),
                ("i", ctypes.c_int64), ("b", ctypes.c_int), ("s", ctypes.c_char_p),
                ("dtype", ctypes.c_int)]


class _TensorRef(ctypes.Structure):
    _fields_ = [("id", ctypes.c_char_p), ("dtype", ctypes.c_int),
                ("shape", ctypes.POINTER(ctypes.c_uint64)), ("rank", ctypes.c_int)]


class _Invocation(ctypes.Structure):
    _fields_ = [("invocation_id", ctypes.c_char_p), ("kernel_name", ctypes.c_char_p),
                ("inputs", ctypes.POINTER(_TensorRef)), ("input_count", ctypes.c_int),
                ("outputs", ctypes.POINTER(_TensorRef)), ("output_count", ctypes.c_int),
                ("attributes", ctypes.POINTER(_Attribute)), ("attribute_count", ctypes.c_int),
                ("deadline_millis", ctypes.c_int64)]


class _Observation(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("kernel", ctypes.c_char * 64),
                ("invocation", ctypes.c_char * 64), ("error", ctypes.c_int)]


class _ProviderMetadata(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("version", ctypes.c_char * 32),
                ("vendor", ctypes.c_char * 64), ("description", ctypes.c_char * 160)]


class _DeviceDescriptor(ctypes.Structure):
    _fields_ = [("id", ctypes.c_char * 32), ("name", ctypes.c_char * 256),
                ("architecture", ctypes.c_char * 64), ("memory_capacity", ctypes.c_uint64),
                ("compute_units", ctypes.c_uint32), ("pressure", ctypes.c_int)]


class _Advertisement(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("operator_name", ctypes.c_char * 48),
                ("operator_family", ctypes.c_char * 32), ("input_dtypes", ctypes.c_uint32),
                ("output_dtypes", ctypes.c_uint32), ("rank", ctypes.c_int),
                ("features", ctypes.c_char * 256), ("conformance_profile", ctypes.c_char * 32),
                ("family", ctypes.c_char * 16), ("device_id", ctypes.c_char * 32),
                ("provider", ctypes.c_char * 128)]


_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_SIGS = {
    "mhip_executor_create": ([_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_P)], ctypes.c_int),
    "mhip_executor_destroy": ([_P], ctypes.c_int),
    "mhip_executor_last_detail": ([], ctypes.c_char_p),
    "mhip_executor_write_tensor": ([_P, ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.c_int, ctypes.c_int, _P, ctypes.c_size_t], ctypes.c_int),
    "mhip_executor_write_tensor_values": ([_P, ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.c_int, ctypes.c_int, _P], ctypes.c_int),
    "mhip_executor_write_zeroed_tensor": ([_P, ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.c_int, ctypes.c_int], ctypes.c_int),
    "mhip_executor_write_weight_tensor": ([_P, ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.c_int, _P, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "mhip_executor_select_greedy_column": ([_P, ctypes.c_char_p, _U64, _P, ctypes.c_uint32, ctypes.c_float, ctypes.POINTER(ctypes.c_int64)], ctypes.c_int),
    "mhip_executor_supports_step_capture": ([_P], ctypes.c_int),
    "mhip_executor_begin_step_capture": ([_P, ctypes.POINTER(ctypes.c_char_p), ctypes.c_int], ctypes.c_int),
    "mhip_executor_end_step_capture": ([_P, ctypes.c_char_p, ctypes.c_size_t], ctypes.c_int),
    "mhip_executor_abort_step_capture": ([_P], ctypes.c_int),
    "mhip_executor_replay_step": ([_P, ctypes.c_char_p, _U64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_P), ctypes.POINTER(_U64), ctypes.c_int], ctypes.c_int),
    "mhip_executor_release_step_capture": ([_P, ctypes.c_char_p], ctypes.c_int),
    "mhip_executor_write_zeroed_kv_store": ([_P, ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.c_int, ctypes.c_int, _U64, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "mhip_executor_read_tensor": ([_P, ctypes.c_char_p, _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "mhip_executor_read_tensor_values": ([_P, ctypes.c_char_p, _P, ctypes.c_size_t], ctypes.c_int),
    "mhip_executor_read_tensor_rows": ([_P, ctypes.c_char_p, _U64, _U64, _P, ctypes.c_size_t], ctypes.c_int),
    "mhip_executor_resident_shape": ([_P, ctypes.c_char_p, ctypes.POINTER(_U64), ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "mhip_executor_release_tensor": ([_P, ctypes.c_char_p], ctypes.c_int),
    "mhip_executor_copy_tensor": ([_P, ctypes.c_char_p, ctypes.c_char_p], ctypes.c_int),
    "mhip_executor_tensor_count": ([_P], _U64),
    "mhip_executor_submit_kernel": ([_P, ctypes.POINTER(_Invocation), ctypes.POINTER(_U64)], ctypes.c_int),
    "mhip_executor_complete_kernel": ([_P, _U64], ctypes.c_int),
    "mhip_executor_execute": ([_P, ctypes.POINTER(_Invocation)], ctypes.c_int),
    "mhip_executor_set_sync_nodes": ([_P, ctypes.c_int], ctypes.c_int),
    "mhip_executor_set_deferred_checks": ([_P, ctypes.c_int], ctypes.c_int),
    "mhip_executor_check": ([_P], ctypes.c_int),
    "mhip_executor_observation_count": ([_P], _U64),
    "mhip_executor_observation": ([_P, _U64, ctypes.POINTER(_Observation)], ctypes.c_int),
    "mhip_provider_create": ([ctypes.c_int, ctypes.c_char_p, ctypes.POINTER(_P)], ctypes.c_int),
    "mhip_provider_destroy": ([_P], ctypes.c_int),
    "mhip_provider_metadata_get": ([_P, ctypes.POINTER(_ProviderMetadata)], ctypes.c_int),
    "mhip_provider_health": ([_P], ctypes.c_int),
    "mhip_provider_device_count": ([_P], ctypes.c_int),
    "mhip_provider_device": ([_P, ctypes.c_int, ctypes.POINTER(_DeviceDescriptor)], ctypes.c_int),
    "mhip_provider_executor": ([_P], _P),
    "mhip_provider_initialize": ([_P], ctypes.c_int),
    "mhip_provider_shutdown": ([_P], ctypes.c_int),
    "mhip_provider_advertisement_count": ([_P], ctypes.c_int),
    "mhip_provider_advertisement": ([_P, ctypes.c_int, ctypes.POINTER(_Advertisement)], ctypes.c_int),
}

_bound = False


def _lib_bound():
    global _bound
    lib = _lib.lib()
    if not _bound:
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _bound = True
    return lib


def _check(code: int) -> None:
    if code != 0:
        raise KernelError(code, _lib_bound().mhip_executor_last_detail().decode())


def _shape(shape: Sequence[int]):
    arr = (ctypes.c_uint64 * max(1, len(shape)))(*[int(s) for s in shape])
    return arr, len(shape)


# ---- invocation model ----
@dataclass
class Float:
    value: float


@dataclass
class Integer:
    value: int


@dataclass
class Boolean:
    value: bool


@dataclass
class String:
    value: str


@dataclass
class DType:
    value: int


@dataclass
class TensorRef:
    id: str
    shape: Sequence[int] = ()
    dtype: int = F32


@dataclass
class KernelInvocation:
    """A Runtime `KernelInvocation`: kernel name, input/output resources, attributes."""
    kernel: str
    inputs: List[TensorRef]
    outputs: List[TensorRef]
    attributes: Dict[str, object] = field(default_factory=dict)
    id: str = "invocation"
    deadline_millis: Optional[int] = None

    def to_c(self):
        keep = []

        def refs(items):
            arr = (_TensorRef * max(1, len(items)))()
            for i, r in enumerate(items):
                shp, rank = _shape(r.shape)
                keep.append(shp)
                arr[i] = _TensorRef(r.id.encode(), r.dtype, shp, rank)
            return arr

        ins, outs = refs(self.inputs), refs(self.outputs)
        attrs = (_Attribute * max(1, len(self.attributes)))()
        for i, (k, v) in enumerate(self.attributes.items()):
            a = _Attribute()
            a.key = k.encode()
            if isinstance(v, bool):
                v = Boolean(v)
            elif isinstance(v, int):
                v = Integer(v)
            elif isinstance(v, float):
                v = Float(v)
            elif isinstance(v, str):
                v = String(v)
            if isinstance(v, Float):
                a.kind, a.f = 0, float(v.value)
            elif isinstance(v, Integer):
                a.kind, a.i = 1, int(v.value)
            elif isinstance(v, Boolean):
                a.kind, a.b = 2, int(bool(v.value))
            elif isinstance(v, String):
                a.kind, a.s = 3, v.value.encode()
            elif isinstance(v, DType):
                a.kind, a.dtype = 4, int(v.value)
            else:
                raise TypeError(f"unsupported attribute value {v!r}")
            attrs[i] = a
        inv = _Invocation(self.id.encode(), self.kernel.encode(), ins, len(self.inputs), outs,
                          len(self.outputs), attrs, len(self.attributes),
                          -1 if self.deadline_millis is None else int(self.deadline_millis))
        keep.extend([ins, outs, attrs])
        return inv, keep


class Executor:
    """`CudaExecutor`-shaped executor: device-resident tensors by resource id."""

    def __init__(self, handle, owner=None):
        self._h = handle
        self._owner = owner  # keeps a Provider alive when it owns the executor

    @classmethod
    def for_device(cls, device, device_id="hip:0", provider_name="magnetar:provider/hip"):
        lib = _lib_bound()
        h = ctypes.c_void_p()
        _lib.check(lib.mhip_executor_create(device.ctx, device_id.encode(),
                                            provider_name.encode(), ctypes.byref(h)))
        ex = cls(h, owner=device)
        ex._owned = True
        return ex

    def close(self):
        if getattr(self, "_owned", False) and self._h:
            _lib_bound().mhip_executor_destroy(self._h)
            self._h = None

    # ---- tensors ----
    def write_tensor(self, id: str, data: np.ndarray, dtype: int = F32) -> None:
        """f32 values for F32; 2-byte bit patterns (uint16) for F16/BF16."""
        data = np.ascontiguousarray(data, dtype=np.float32 if dtype == F32 else np.uint16)
        shp, rank = _shape(data.shape)
        _check(_lib_bound().mhip_executor_write_tensor(self._h, id.encode(), shp, rank, dtype,
                                                       data.ctypes.data_as(_P), data.nbytes))

    def write_tensor_values(self, id: str, values: np.ndarray, dtype: int) -> None:
        values = np.ascontiguousarray(values, dtype=np.float32)
        shp, rank = _shape(values.shape)
        _check(_lib_bound().mhip_executor_write_tensor_values(self._h, id.encode(), shp, rank,
                                                              dtype, values.ctypes.data_as(_P)))

    def write_zeroed_tensor(self, id: str, shape: Sequence[int], dtype: int = F32) -> None:
        shp, rank = _shape(shape)
        _check(_lib_bound().mhip_executor_write_zeroed_tensor(self._h, id.encode(), shp, rank, dtype))

    def write_weight_tensor(self, id: str, values: np.ndarray) -> bool:
        """A weight (src/executor.rs:384-399): stored compact as bf16 bits when it
        is a matrix of >= 65536 exact bf16 values; returns whether it was."""
        v = np.ascontiguousarray(values, np.float32)
        shp, rank = _shape(v.shape)
        compact = ctypes.c_int(0)
        _check(_lib_bound().mhip_executor_write_weight_tensor(
            self._h, id.encode(), shp, rank, v.ctypes.data_as(_P), ctypes.byref(compact)))
        return bool(compact.value)

    def write_zeroed_kv_store(self, id: str, shape: Sequence[int], precision: int = KV_F32,
                              head_dimension: int = 0) -> bool:
        """A zeroed KV store (src/executor.rs:560-602). True when stored; the
        quantized precisions are declined (False) and nothing is written."""
        shp, rank = _shape(shape)
        stored = ctypes.c_int(0)
        _check(_lib_bound().mhip_executor_write_zeroed_kv_store(
            self._h, id.encode(), shp, rank, precision, head_dimension, ctypes.byref(stored)))
        return bool(stored.value)

    def resident_shape(self, id: str):
        shp = (ctypes.c_uint64 * 8)()
        rank, dtype = ctypes.c_int(0), ctypes.c_int(0)
        _check(_lib_bound().mhip_executor_resident_shape(self._h, id.encode(), shp,
                                                         ctypes.byref(rank), ctypes.byref(dtype)))
        return tuple(shp[i] for i in range(rank.value)), dtype.value

    def read_tensor(self, id: str) -> np.ndarray:
        """The stored data: f32 values, or uint16 bit patterns for half tensors."""
        shape, dtype = self.resident_shape(id)
        out = np.empty(shape, np.float32 if dtype == F32 else np.uint16)
        written = ctypes.c_size_t(0)
        _check(_lib_bound().mhip_executor_read_tensor(self._h, id.encode(), out.ctypes.data_as(_P),
                                                      out.nbytes, ctypes.byref(written)))
        return out

    def read_tensor_values(self, id: str) -> np.ndarray:
        shape, _ = self.resident_shape(id)
        out = np.empty(shape, np.float32)
        _check(_lib_bound().mhip_executor_read_tensor_values(self._h, id.encode(),
                                                             out.ctypes.data_as(_P), out.size))
        return out

    def read_tensor_rows(self, id: str, row_begin: int, row_count: int) -> np.ndarray:
        shape, _ = self.resident_shape(id)
        width = int(np.prod(shape[1:], dtype=np.int64)) if len(shape) > 1 else 1
        out = np.empty((row_count,) + tuple(shape[1:]), np.float32)
        _check(_lib_bound().mhip_executor_read_tensor_rows(self._h, id.encode(), row_begin,
                                                           row_count, out.ctypes.data_as(_P),
                                                           row_count * width))
        return out

    def release_tensor(self, id: str) -> None:
        _check(_lib_bound().mhip_executor_release_tensor(self._h, id.encode()))

    def copy_tensor(self, src: str, dst: str) -> None:
        _check(_lib_bound().mhip_executor_copy_tensor(self._h, src.encode(), dst.encode()))

    def tensor_count(self) -> int:
        return int(_lib_bound().mhip_executor_tensor_count(self._h))

    # ---- dispatch ----
    def submit_kernel(self, inv: KernelInvocation) -> int:
        c, keep = inv.to_c()
        handle = ctypes.c_uint64(0)
        _check(_lib_bound().mhip_executor_submit_kernel(self._h, ctypes.byref(c), ctypes.byref(handle)))
        return handle.value

    def complete_kernel(self, handle: int) -> None:
        """Raises KernelError when the Kernel failed."""
        _check(_lib_bound().mhip_executor_complete_kernel(self._h, handle))

    def execute(self, inv: KernelInvocation) -> None:
        self.complete_kernel(self.submit_kernel(inv))

    def select_greedy_column(self, logits: str, row: int = 0, excluded=(),
                             temperature: float = 0.0):
        """The greedy column of `logits` row `row` (src/executor.rs:2549-2564), or
        None when no column is eligible or the selection fails, as the
        reference's Option."""
        self.check()  # a deferred failure raises rather than reading as None
        flat = [int(v) for r in excluded for v in (r[0], r[1])]
        ranges = (ctypes.c_uint64 * max(1, len(flat)))(*flat)
        col = ctypes.c_int64(-1)
        code = _lib_bound().mhip_executor_select_greedy_column(
            self._h, logits.encode(), row, ranges, len(flat) // 2, temperature, ctypes.byref(col))
        return None if code != 0 or col.value < 0 else int(col.value)

    # ---- step capture (src/executor.rs:177-336) ----
    def supports_step_capture(self) -> bool:
        return bool(_lib_bound().mhip_executor_supports_step_capture(self._h))

    def begin_step_capture(self, advancing_attributes: Sequence[str] = ()) -> None:
        names = (ctypes.c_char_p * max(1, len(advancing_attributes)))(
            *[a.encode() for a in advancing_attributes])
        _check(_lib_bound().mhip_executor_begin_step_capture(self._h, names,
                                                             len(advancing_attributes)))

    def end_step_capture(self) -> str:
        """Instantiates the captured step and runs it once; returns its id."""
        buf = ctypes.create_string_buffer(256)
        _check(_lib_bound().mhip_executor_end_step_capture(self._h, buf, 256))
        return buf.value.decode()

    def abort_step_capture(self) -> None:
        _check(_lib_bound().mhip_executor_abort_step_capture(self._h))

    def replay_step(self, capture_id: str, offset: int = 0, inputs=None) -> None:
        """Writes `inputs` ({resource id: f32 array}) into the step's buffers and
        runs it with every advancing attribute increased by `offset`."""
        items = [(k, np.ascontiguousarray(v, np.float32).ravel()) for k, v in (inputs or {}).items()]
        n = len(items)
        ids = (ctypes.c_char_p * max(1, n))(*[k.encode() for k, _ in items])
        ptrs = (_P * max(1, n))(*[a.ctypes.data for _, a in items])
        lens = (_U64 * max(1, n))(*[a.size for _, a in items])
        _check(_lib_bound().mhip_executor_replay_step(self._h, capture_id.encode(), offset, ids,
                                                      ptrs, lens, n))

    def release_step_capture(self, capture_id: str) -> None:
        _check(_lib_bound().mhip_executor_release_step_capture(self._h, capture_id.encode()))

    def set_sync_nodes(self, enabled: bool) -> None:
        _lib.check(_lib_bound().mhip_executor_set_sync_nodes(self._h, int(enabled)))

    def set_deferred_checks(self, enabled: bool) -> None:
        """Enabled, embedding and softmax dispatches no longer wait for their
        failure flags; the next read, greedy selection, capture start or
        check() reads them once and raises the deferred failure. Disabling
        checks what is pending."""
        _check(_lib_bound().mhip_executor_set_deferred_checks(self._h, int(enabled)))

    def check(self) -> None:
        """Raises the failure of any dispatch whose check was deferred."""
        _check(_lib_bound().mhip_executor_check(self._h))

    def observations(self):
        lib = _lib_bound()
        out = []
        for i in range(int(lib.mhip_executor_observation_count(self._h))):
            o = _Observation()
            _lib.check(lib.mhip_executor_observation(self._h, i, ctypes.byref(o)))
            out.append((OBSERVATIONS.get(o.kind, o.kind), o.kernel.decode(), o.invocation.decode(),
                        KERNEL_ERRORS.get(o.error, o.error)))
        return out


@dataclass
class Advertisement:
    name: str
    operator_name: str
    operator_family: str
    input_dtypes: List[int]
    output_dtypes: List[int]
    rank: Optional[int]
    features: List[str]
    conformance_profile: str
    family: str
    device_id: str
    provider: str


class Provider:
    """`CudaProvider`-shaped facade: never fails construction for lack of hardware."""

    def __init__(self, ordinal: int = 0, name: str = "magnetar:provider/hip"):
        lib = _lib_bound()
        h = ctypes.c_void_p()
        _lib.check(lib.mhip_provider_create(ordinal, name.encode(), ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            _lib_bound().mhip_provider_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def metadata(self) -> dict:
        m = _ProviderMetadata()
        _lib.check(_lib_bound().mhip_provider_metadata_get(self._h, ctypes.byref(m)))
        return {"name": m.name.decode(), "version": m.version.decode(),
                "vendor": m.vendor.decode(), "description": m.description.decode()}

    def is_available(self) -> bool:
        return self.health() != "Unavailable"

    def health(self) -> str:
        return HEALTH[_lib_bound().mhip_provider_health(self._h)]

    def devices(self) -> list:
        lib = _lib_bound()
        out = []
        for i in range(lib.mhip_provider_device_count(self._h)):
            d = _DeviceDescriptor()
            _lib.check(lib.mhip_provider_device(self._h, i, ctypes.byref(d)))
            out.append({"id": d.id.decode(), "name": d.name.decode(),
                        "architecture": d.architecture.decode(),
                        "memory_capacity": d.memory_capacity, "compute_units": d.compute_units,
                        "pressure": d.pressure})
        return out

    def kernel_advertisements(self) -> List[Advertisement]:
        lib = _lib_bound()
        out = []
        for i in range(lib.mhip_provider_advertisement_count(self._h)):
            a = _Advertisement()
            _lib.check(lib.mhip_provider_advertisement(self._h, i, ctypes.byref(a)))
            dts = lambda mask: [d for d in (F32, F16, BF16) if mask & (1 << d)]
            out.append(Advertisement(a.name.decode(), a.operator_name.decode(),
                                     a.operator_family.decode(), dts(a.input_dtypes),
                                     dts(a.output_dtypes), a.rank or None,
                                     [f for f in a.features.decode().split(",") if f],
                                     a.conformance_profile.decode(), a.family.decode(),
                                     a.device_id.decode(), a.provider.decode()))
        return out

    def execution_api(self) -> Optional[Executor]:
        h = _lib_bound().mhip_provider_executor(self._h)
        return Executor(ctypes.c_void_p(h), owner=self) if h else None

    def initialize(self) -> None:
        _lib.check(_lib_bound().mhip_provider_initialize(self._h))

    def shutdown(self) -> None:
        _lib.check(_lib_bound().mhip_provider_shutdown(self._h))
