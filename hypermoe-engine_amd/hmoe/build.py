"""Build driver for the MI355X MoE-block engine.

Compiles, in tree (so the shared objects travel with the source tree):
  lib/libhm_kernels.so  HIP kernels + C ABI (include/hm_moe.h), gfx950
  lib/libhm_synth.so    seeded synthetic-input generator (host C)
  lib/libhm_host.so     C++20 host layer (HipBackend, HipTensorBackend,
                        HipMoEBlock) over the C ABI
and, as test infrastructure, oracle/libhm_oracle.so and (where the reference
tree is mounted) oracle/_ref/libhm_ref.so.

Every HIP translation unit is built with -ffp-contract=off (FMAs only where a
kernel asks for one explicitly) and with packed FP32 instructions disabled.
Sources with hand-written memory statements (CHECKED_SOURCES: loads the
compiler does not track, LDS-DMA loads that set M0) are assembled from a
saved listing that hmoe.isa_check verifies first: no register of an
untracked load is touched before a wait completes it, the compiler's own
code leaves M0 alone, and the hand-written blocks hold only the memory
forms the check understands.
"""
from __future__ import annotations

import concurrent.futures as _futures
import os
import shutil
import subprocess
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent          # hypermoe-engine_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
HOST = PKG_ROOT / "host"
LIB = PKG_ROOT / "lib"
OBJ = PKG_ROOT / "_build"
INCLUDE = REPO_ROOT / "include"
ORACLE = REPO_ROOT / "oracle"
REFERENCE = Path(os.environ.get("HM_REFERENCE_ROOT", "/root/reference"))

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
KERNEL_SOURCES = ["hm_runtime.hip", "hm_router.hip", "hm_gemm.hip", "hm_gemm_mfma.hip",
                  "hm_gemm_f32_mfma.hip", "hm_gemv.hip", "hm_block.hip", "hm_noalloc.hip"]
# Per-source flags.  The FP64 router MFMAs keep their accumulators in VGPRs
# (otherwise the compiler copies them to AGPRs and back on every K chunk).
SOURCE_FLAGS = {"hm_router.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
                "hm_gemm_f32_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
# Sources with hand-written memory statements: register loads the compiler
# does not track (hm_gemm_mfma.hip) and LDS-DMA loads that set M0 (all three).
CHECKED_SOURCES = {"hm_gemm_mfma.hip", "hm_router.hip", "hm_gemm_f32_mfma.hip"}
HOST_SOURCES = ["hip_backend.cpp", "hip_tensor_backend.cpp", "moe_block.cpp", "artefact.cpp"]

KERNELS_SO = LIB / "libhm_kernels.so"
SYNTH_SO = LIB / "libhm_synth.so"
HOST_SO = LIB / "libhm_host.so"
ORACLE_SO = ORACLE / "libhm_oracle.so"
REF_SO = ORACLE / "_ref" / "libhm_ref.so"


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    res = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}")


def _quiet_filter(text: str) -> str:
    # the feature warning of the host pass, and the note on the M0 clobber of
    # the LDS-DMA statements (isa_check verifies that the compiled code keeps
    # nothing else in M0)
    return "\n".join(l for l in text.splitlines()
                     if "packed-fp32-ops" not in l and "Reserved registers on the clobber list" not in l
                     and "clobber list contains reserved registers" not in l
                     and not l.endswith("warnings generated."))


def _device_listing(obj: Path) -> Path:
    return obj.with_name(f"{obj.stem}-hip-amdgcn-amd-amdhsa-{ARCH}.s")


def _compile_hip(src: Path, obj: Path) -> str:
    checked = src.name in CHECKED_SOURCES
    # -save-temps=obj: the object is assembled from the listing that is checked
    extra = ["-save-temps=obj"] if checked else []
    cmd = [HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}")
    if checked:
        from hmoe import isa_check
        listing = _device_listing(obj)
        for tmp in obj.parent.glob(f"{obj.stem}-*"):
            if tmp != listing:
                tmp.unlink()
        for tmp in obj.parent.glob(f"{obj.stem}.hip-*"):
            tmp.unlink()
        problems = isa_check.check_file(listing)
        if problems:
            obj.unlink(missing_ok=True)
            raise RuntimeError(f"{src.name}: the compiled code breaks the rules of its "
                               "hand-written memory statements (hmoe.isa_check):\n"
                               + "\n".join(problems[:20]))
    return _quiet_filter(res.stdout)


def build_kernels(jobs: int = 4) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    LIB.mkdir(parents=True, exist_ok=True)
    srcs = [CSRC / s for s in KERNEL_SOURCES]
    objs = [OBJ / (s.stem + ".o") for s in srcs]
    with _futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for log in pool.map(_compile_hip, srcs, objs):
            if log.strip():
                print(log)
    tmp = KERNELS_SO.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, KERNELS_SO)
    return KERNELS_SO


def build_synth() -> Path:
    LIB.mkdir(parents=True, exist_ok=True)
    tmp = SYNTH_SO.with_suffix(".so.tmp")
    _run(["gcc", "-std=c11", "-O3", "-ffp-contract=off", "-fPIC", "-shared", "-Wall",
          "-o", str(tmp), str(HOST / "hm_synth.c"), "-lm", "-lpthread"])
    os.replace(tmp, SYNTH_SO)
    return SYNTH_SO


def build_host() -> Path | None:
    srcs = [HOST / s for s in HOST_SOURCES]
    if not all(s.exists() for s in srcs):
        return None
    LIB.mkdir(parents=True, exist_ok=True)
    tmp = HOST_SO.with_suffix(".so.tmp")
    # host C++ only: every device call goes through the C ABI of libhm_kernels.so
    _run(["g++", "-std=c++20", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", f"-I{INCLUDE}",
          "-o", str(tmp), *map(str, srcs), f"-L{LIB}", "-lhm_kernels", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOST_SO)
    return HOST_SO


def build_oracle(with_reference: bool = True) -> None:
    """Test infrastructure: the C restatement, and the reference build where
    the reference tree is present (it never is on the GPU box)."""
    _run(["make", "-s", "-C", str(ORACLE)])
    if with_reference and (REFERENCE / "src").is_dir():
        _run(["make", "-s", "-j8", "-C", str(ORACLE), "ref", f"REF_ROOT={REFERENCE}"])


def build_all(jobs: int = 4) -> None:
    build_kernels(jobs)
    build_synth()
    build_host()
    build_oracle()


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)
    for p in (KERNELS_SO, SYNTH_SO, HOST_SO):
        p.unlink(missing_ok=True)


if __name__ == "__main__":
    build_all()
    print("built", KERNELS_SO, SYNTH_SO)
