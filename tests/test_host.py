"""Host-side checks that run without a GPU: the C ABI library loads and exports
every function include/magnetar_hip.h declares, and the Provider's
"no hardware" contract (reference src/tests.rs:73-165): construction never
fails, health is Unavailable, no devices, no advertisements, no executor.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "magnetar_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mhip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for required in ["mhip_add_f32", "mhip_mul_f32", "mhip_bias_add_f32", "mhip_mul_scalar_f32",
                     "mhip_silu_f32", "mhip_silu_mul_f32", "mhip_embedding_f32",
                     "mhip_rmsnorm_f32", "mhip_rope_f32", "mhip_softmax_rows_f32",
                     "mhip_matmul_f32", "mhip_attention_f32", "mhip_add_half", "mhip_mul_half",
                     "mhip_executor_submit_kernel", "mhip_executor_complete_kernel",
                     "mhip_provider_create"]:
        assert required in names


def test_library_exports_every_declared_function():
    import magnetar_hip
    lib = ctypes.CDLL(magnetar_hip._lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_bindings_cover_the_abi():
    from magnetar_hip import _lib, executor, decoder
    bound = set(_lib.SIGNATURES) | set(executor._SIGS) | set(decoder.SIGNATURES)
    assert set(declared_functions()) <= bound


def test_status_names_match_the_reference_categories():
    import magnetar_hip
    lib = magnetar_hip.lib()
    names = [lib.mhip_status_name(i).decode() for i in range(10)]
    # CudaErrorCode (src/error.rs:15-42), in order after Ok.
    assert names == ["Ok", "ShapeUnsupported", "DTypeUnsupported", "LayoutUnsupported",
                     "ExecutionFailed", "OutOfDeviceMemory", "CompilationFailed",
                     "DriverFailed", "DeviceUnavailable", "CaptureUnsupported"]


def _gpu_present():
    import magnetar_hip
    return magnetar_hip.device_count() > 0


def test_provider_is_gracefully_unavailable_without_a_gpu():
    import magnetar_hip
    if _gpu_present():
        pytest.skip("a GPU is present: covered by the gpu tests")
    with magnetar_hip.Provider() as provider:
        assert provider.metadata()["name"] == "magnetar:provider/hip"
        assert provider.metadata()["version"] == "0.1.0"
        assert provider.health() == "Unavailable"
        assert provider.devices() == []
        assert provider.kernel_advertisements() == []
        assert provider.execution_api() is None
        provider.initialize()
        provider.shutdown()


def test_second_ordinal_is_unavailable_not_an_error():
    """for_device on an ordinal with no device (src/tests.rs:167-255)."""
    import magnetar_hip
    with magnetar_hip.Provider(ordinal=7, name="magnetar:provider/hip-7") as provider:
        assert provider.metadata()["name"] == "magnetar:provider/hip-7"
        assert provider.health() == "Unavailable"
        assert provider.devices() == []


def test_device_context_fails_cleanly_without_a_gpu():
    import magnetar_hip
    if _gpu_present():
        pytest.skip("a GPU is present")
    with pytest.raises(magnetar_hip.MagnetarHipError) as err:
        magnetar_hip.Device(0)
    assert err.value.code == "DeviceUnavailable"


def test_kernel_entry_points_refuse_a_null_context():
    """No compute without a device: every kernel entry checks its context first."""
    import magnetar_hip
    lib = magnetar_hip.lib()
    assert lib.mhip_add_f32(None, None, None, None, 16) == 8
    assert lib.mhip_matmul_f32(None, None, None, None, 2, 2, 2, 0, 0, None, 0) == 8
    assert lib.mhip_sync(None) == 8


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 prints why and exits non-zero
    before touching a device."""
    import json
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    done = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert done.returncode != 0
    line = json.loads(done.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]
