"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU
only): the C++ host layer (HipBackend, HipTensorBackend, HipMoEBlock and the
packed-artefact reader, which parses untrusted index and manifest files),
the host side of the C ABI library and the synthetic-input generator are
rebuilt with -fsanitize=address,undefined (host code only: the device code
objects are unchanged and never run here) into a temporary directory, then

  - the C++ host-layer test program runs its CPU mode on them, and
  - tests/test_artefact.py and tests/test_capi_host.py run against them in a
    Python process with the sanitizer runtimes preloaded.

Any sanitizer report ends the run with a non-zero status (halt_on_error);
leak checking is off (the Python interpreter itself does not free
everything at exit)."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "hypermoe-engine_amd"
sys.path.insert(0, str(PKG))

from hmoe import build as B  # noqa: E402

# ROCm's clang throughout (hipcc's host objects need its sanitizer runtime,
# shared so that one copy serves every library and the Python process)
CLANG = "/opt/rocm/llvm/bin/clang"
CLANGXX = "/opt/rocm/llvm/bin/clang++"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
       "-fno-omit-frame-pointer", "-shared-libsan"]
ENV = {"ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
       "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _asan_runtime() -> str:
    return subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"],
                          capture_output=True, text=True).stdout.strip()


def _run(cmd, **kw):
    res = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert res.returncode == 0, f"{' '.join(map(str, cmd[:6]))} ...\n{res.stdout}\n{res.stderr}"
    return res


@pytest.fixture(scope="module")
def sanitized(tmp_path_factory):
    """libhm_kernels.so (host code sanitized), libhm_host.so, libhm_synth.so
    and the C++ test program, all in one temporary directory."""
    d = tmp_path_factory.mktemp("san")
    rt = [f"-Wl,-rpath,{Path(_asan_runtime()).parent}"]
    hip_host_san = [a for f in SAN for a in ("-Xarch_host", f)]
    objs = []
    procs = []
    for src in B.KERNEL_SOURCES:
        obj = d / (Path(src).stem + ".o")
        cmd = [B.HIPCC, *B.HIP_FLAGS, *B.SOURCE_FLAGS.get(src, []), *hip_host_san, "-g",
               "-c", str(B.CSRC / src), "-o", str(obj)]
        procs.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                       text=True), cmd))
        objs.append(obj)
    for p, cmd in procs:
        out, _ = p.communicate()
        assert p.returncode == 0, f"{' '.join(cmd[-4:])}\n{out}"
    kern = d / "libhm_kernels.so"
    _run([B.HIPCC, f"--offload-arch={B.ARCH}", "-shared", "-fPIC", *hip_host_san, *rt, "-o",
          str(kern), *map(str, objs)])
    _run([CLANG, "-std=c11", "-O1", "-g", "-fPIC", "-shared", *SAN, *rt, "-o",
          str(d / "libhm_synth.so"), str(B.HOST / "hm_synth.c"), "-lm", "-lpthread"])
    _run([CLANGXX, "-std=c++20", "-O1", "-g", "-fPIC", "-shared", *SAN, f"-I{B.INCLUDE}", "-o",
          str(d / "libhm_host.so"), *[str(B.HOST / s) for s in B.HOST_SOURCES], f"-L{d}",
          "-lhm_kernels", f"-Wl,-rpath,{d}", *rt])
    B.build_oracle(with_reference=False)
    _run([CLANGXX, "-std=c++20", "-O1", "-g", *SAN, f"-I{B.INCLUDE}", f"-I{B.ORACLE}", "-o",
          str(d / "test_host"), str(REPO / "tests" / "cpp" / "test_host.cpp"), f"-L{d}",
          "-lhm_host", "-lhm_kernels", "-lhm_synth", f"-L{B.ORACLE}", "-lhm_oracle",
          f"-Wl,-rpath,{d}", f"-Wl,-rpath,{B.ORACLE}", *rt])
    return d


def test_cpp_host_layer_cpu_sanitized(sanitized):
    res = _run([str(sanitized / "test_host"), "cpu"], timeout=300,
               env={**os.environ, **ENV})
    assert " 0 failures" in res.stdout
    assert "AddressSanitizer" not in res.stderr and "runtime error" not in res.stderr


def test_python_host_abi_sanitized(sanitized):
    """The artefact reader/writer and the C ABI host checks, with the
    sanitized libraries in place of the built ones."""
    preload = _asan_runtime()
    script = (
        "import sys; sys.path.insert(0, %r); from pathlib import Path\n"
        "from hmoe import build as B\n"
        "d = Path(%r)\n"
        "B.HOST_SO = d / 'libhm_host.so'; B.KERNELS_SO = d / 'libhm_kernels.so';"
        " B.SYNTH_SO = d / 'libhm_synth.so'\n"
        "import pytest\n"
        "sys.exit(pytest.main(['-q', '-x', '-m', 'not gpu', '-p', 'no:cacheprovider',"
        " '-p', 'no:xdist', %r, %r]))\n"
    ) % (str(PKG), str(sanitized), str(REPO / "tests" / "test_artefact.py"),
         str(REPO / "tests" / "test_capi_host.py"))
    res = _run([sys.executable, "-c", script], timeout=600, cwd=str(REPO / "tests"),
               env={**os.environ, **ENV, "LD_PRELOAD": preload})
    assert "passed" in res.stdout
    assert "AddressSanitizer" not in res.stderr and "runtime error" not in res.stderr
