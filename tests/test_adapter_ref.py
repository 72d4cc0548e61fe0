"""The reference-side adapter (hypermoe-engine_amd/integration/HipMoEAdapter)
compiled against the reference's own headers, with the reference's Tensor,
Shape, TensorView, ExpertBatch and DeviceBuffer sources compiled where they
lie, and linked with libhm_host.so: toReference on a host-built
hm::BatchLayerExecutionResult gives a hypermoe::runtime::BatchLayerExecutionResult
(src/core/runtime/MoERuntime.hpp:33-39) equal member by member, toHm keeps a
reference view's storage, and HipComputeBackend serves through the
reference's ComputeBackend (src/backend/Backend.hpp:36-71).  A second build,
against a copy of the reference's sources with the HIP enumerators added
(integration/reference_enums.py), converts HIP-device tensors.  Runs where
the reference tree is mounted (the build container), skipped elsewhere."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
REF = Path(os.environ.get("HM_REFERENCE_ROOT", "/root/reference"))
LIB = REPO / "hypermoe-engine_amd" / "lib"

pytestmark = pytest.mark.skipif(not (REF / "src" / "tensor" / "Tensor.cpp").exists(),
                                reason="reference tree not mounted")

REF_SOURCES = ["src/tensor/Tensor.cpp", "src/tensor/Shape.cpp", "src/tensor/TensorView.cpp",
               "src/experts/ExpertBatch.cpp", "src/backend/Backend.cpp"]


def _build_and_run(ref: Path, exe: Path, defines=()) -> str:
    cmd = ["g++", "-std=c++20", "-O1", "-Wall", "-Werror", *defines,
           f"-I{ref / 'src'}", f"-I{ref / 'src' / 'core'}", f"-I{ref / 'include'}",
           f"-I{REPO / 'include'}", f"-I{REPO / 'hypermoe-engine_amd' / 'integration'}",
           str(REPO / "tests" / "cpp" / "adapter_check.cpp"),
           str(REPO / "hypermoe-engine_amd" / "integration" / "HipMoEAdapter.cpp"),
           *[str(ref / s) for s in REF_SOURCES],
           f"-L{LIB}", "-lhm_host", "-lhm_kernels", f"-Wl,-rpath,{LIB}", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stdout + build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    return run.stdout


def test_adapter_against_reference_interfaces(tmp_path):
    if not (LIB / "libhm_host.so").exists():
        pytest.skip("libhm_host.so not built")
    out = _build_and_run(REF, tmp_path / "adapter_check")
    assert "adapter ok" in out


def test_adapter_device_tensors_with_reference_enums(tmp_path):
    """The device path: a copy of the reference's sources with the three
    enumerator edits of integration/reference_enums.py (HIP in DeviceType,
    isValid and toString; Hip in BackendKind) accepts the HIP-device tensors
    toReference produces, with device, storage and shape kept."""
    if not (LIB / "libhm_host.so").exists():
        pytest.skip("libhm_host.so not built")
    import shutil
    import sys
    ref = tmp_path / "ref"
    shutil.copytree(REF / "src", ref / "src")
    if (REF / "include").is_dir():
        shutil.copytree(REF / "include", ref / "include")
    sys.path.insert(0, str(REPO / "hypermoe-engine_amd" / "integration"))
    import reference_enums
    reference_enums.apply(ref)
    assert "HIP = 2" in (ref / "src" / "tensor" / "Tensor.hpp").read_text()
    out = _build_and_run(ref, tmp_path / "adapter_check_dev", ["-DHM_ADAPTER_HIP_ENUMS"])
    assert "adapter device tensors ok" in out and "adapter ok" in out
