"""CPU: every gfx950 kernel of the built library runs without scratch memory.

A kernel that spills registers or copies a by-value argument to private
memory (scratch) runs several times slower and no parity test notices. This
reads the kernel descriptors of the library's own device code objects (the
`.hip_fatbin` section of each object under `_build/`, unbundled with the ROCm
LLVM tools) and requires, per kernel, a zero private segment and no VGPR
spills. SGPR spills are allowed while the private segment stays zero: they
then live in spare VGPR lanes (register moves, not memory).
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "magnetar-provider-cuda_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
TOOLS = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")]
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _objects():
    if not os.path.isdir(BUILD):
        return []
    return sorted(os.path.join(BUILD, f) for f in os.listdir(BUILD)
                  if f.endswith(".o") and not f.endswith(".cpp.o"))


def _kernel_resources(obj, tmp):
    """{kernel name: {field: value}} from the object's gfx950 code object."""
    base = os.path.join(tmp, os.path.basename(obj))
    subprocess.run([TOOLS[0], f"--dump-section=.hip_fatbin={base}.fatbin", obj, f"{base}.host"],
                   check=True, capture_output=True)
    subprocess.run([TOOLS[1], "--unbundle", "--type=o", f"--targets={TARGET}",
                    f"--input={base}.fatbin", f"--output={base}.co"], check=True, capture_output=True)
    notes = subprocess.run([TOOLS[2], "--notes", f"{base}.co"], check=True, capture_output=True,
                           text=True).stdout
    kernels, current = {}, None
    for line in notes.splitlines():
        m = re.match(r"\s+\.name:\s+(\S+)", line)
        if m:
            current = kernels.setdefault(m.group(1), {})
            continue
        m = re.match(r"\s+\.(private_segment_fixed_size|vgpr_spill_count|sgpr_spill_count):\s+(\d+)", line)
        if m and current is not None:
            current[m.group(1)] = int(m.group(2))
    return kernels


@pytest.mark.skipif(not all(os.path.exists(t) for t in TOOLS), reason="ROCm LLVM tools absent")
def test_no_kernel_uses_scratch():
    objects = _objects()
    if not objects:
        pytest.skip("library not built (make -C magnetar-provider-cuda_amd)")
    tmp = tempfile.mkdtemp()
    try:
        offenders, count = [], 0
        for obj in objects:
            for name, fields in _kernel_resources(obj, tmp).items():
                count += 1
                if any(fields.get(f, 0) for f in ("private_segment_fixed_size", "vgpr_spill_count")):
                    offenders.append(f"{os.path.basename(obj)}: {name} {fields}")
        assert count > 20, f"only {count} kernels found"
        assert not offenders, "kernels using scratch:\n" + "\n".join(offenders)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def test_every_launch_goes_through_the_recording_wrapper():
    """Step capture records the launches made through mhip::launch (common.hpp)
    and re-issues them on replay; a launch made any other way would run
    during a capture instead of being recorded. Only the wrapper and the
    replay itself (runtime.hip) call the HIP launch API."""
    import glob
    csrc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "magnetar-provider-cuda_amd", "csrc")
    found = []
    for path in sorted(glob.glob(os.path.join(csrc, "*"))):
        text = open(path).read()
        name = os.path.basename(path)
        raw = text.count("hipLaunchKernelGGL") + text.count("<<<") + text.count("hipLaunchKernel(")
        allowed = {"common.hpp": 1, "runtime.hip": 1}.get(name, 0)
        if raw != allowed:
            found.append((name, raw))
    assert not found, f"launches outside mhip::launch: {found}"
