"""The C++20 host layer (HipBackend, HipTensorBackend, HipMoEBlock) through
its own C++ test program, tests/cpp/test_host.cpp (built by
__graft_entry__.build() via tests/cpp/Makefile)."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "_bin" / "test_host"


def _run(mode: str, timeout: int) -> None:
    assert BIN.exists(), f"{BIN} is not built: run __graft_entry__.build()"
    res = subprocess.run([str(BIN), mode], capture_output=True, text=True, timeout=timeout)
    print(res.stdout)
    print(res.stderr)
    assert res.returncode == 0, f"C++ host tests ({mode}) failed:\n{res.stdout}\n{res.stderr}"
    assert " 0 failures" in res.stdout


def test_cpp_host_layer_cpu():
    """Argument checks, error categories, lifetimes and the no-device
    behaviour of the backend (no GPU is visible to this process)."""
    _run("cpu", 120)


@pytest.mark.gpu
def test_cpp_host_layer_gpu():
    """Device backend, tensor backend ops against the oracle, and
    HipMoEBlock::executeBatch bit-exact against the limb oracle and within
    1e-4 of the reference W8A32 path."""
    print("[gpu] C++ host layer", flush=True)
    _run("gpu", 300)
