"""The C ABI without a GPU: libhm_kernels.so loads, exports every function
include/hm_moe.h declares, and its host-only logic (launch plans, workspace
sizes, the INT8 packer, argument validation) behaves.  CPU only."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact
from hmoe import capi

HEADER = Path(__file__).resolve().parent.parent / "include" / "hm_moe.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_the_binding_knows():
    names = declared_functions()
    assert len(names) > 30
    assert set(names) == set(capi.SIGNATURES), set(names) ^ set(capi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.hm_abi_version() == 1
    assert lib.hm_status_string(1) == b"invalid argument"


def test_library_exports_nothing_undeclared():
    """The kernel library's dynamic symbol table holds no hm_* entry point
    beyond the header's (internal helpers are hidden)."""
    import shutil
    import subprocess
    if shutil.which("nm") is None:
        pytest.skip("nm is not installed")
    out = subprocess.run(["nm", "-D", "--defined-only", str(capi.lib_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = {f.split()[-1] for f in out.splitlines() if f.split() and f.split()[-1].startswith("hm_")}
    extra = sorted(exported - set(declared_functions()))
    assert not extra, extra


def test_plan_known_answers():
    """tests/phase23_tests.cpp:34-46 (mode, partitions, scratch)."""
    def plan(r, k, n, mode=0):
        p = capi.HmInt8GemmPlan()
        rc = capi.status("hm_plan_int8_gemm", r, k, n, mode, C.byref(p))
        return rc, p
    rc, p = plan(1, 2048, 768)
    assert rc == 0 and p.implementation == 2 and p.partitions == 4 and p.scratch_elements == 3072
    rc, p = plan(1, 768, 2048)
    assert p.partitions == 2 and p.implementation == 2
    rc, p = plan(1, 2048, 768, 1)
    assert p.implementation == 1 and p.blocks == 3
    assert plan(1, 8, 8)[1].implementation == 1
    assert plan(2, 257, 65)[1].scratch_elements == 0
    assert plan(1, 8193, 65)[1].partitions == 8
    assert plan(0, 10, 10)[0] == capi.HM_ERR_INVALID
    assert plan(2, 2 ** 62, 4)[0] == capi.HM_ERR_OVERFLOW
    assert plan(1, 1, 1, 99)[0] == capi.HM_ERR_INVALID


def test_host_packer_matches_reference_quantiser():
    """hm_quantize_int8_host == Quantization.cpp:45-79 (through the oracle)."""
    rng = np.random.default_rng(0)
    for w in [(0.02 * rng.standard_normal(5000)).astype(np.float32),
              np.array([-2.0, -0.25, 0.0, 0.75, 2.0], np.float32), np.zeros(7, np.float32),
              np.array([0.5, -0.5, 1.5, 2.5, -2.5, 127.0], np.float32)]:
        q = np.empty(w.shape, np.int8)
        s, z, e = C.c_float(), C.c_int32(), C.c_float()
        capi.call("hm_quantize_int8_host", w.ctypes.data, w.size, q.ctypes.data, C.byref(s),
                  C.byref(z), C.byref(e))
        q2, s2, z2, e2 = O.quantize_int8(w)
        assert_bitexact(q, q2, "packed bytes")
        assert (s.value, z.value, e.value) == (s2, z2, e2)
    bad = np.array([1.0, np.nan], np.float32)
    assert capi.status("hm_quantize_int8_host", bad.ctypes.data, 2, bad.ctypes.data, None, None,
                       None) == capi.HM_ERR_INVALID


def test_workspace_and_layer_sizes():
    lib = capi.load()
    assert lib.hm_packed_layer_bytes(128, 2048, 768, capi.HM_DTYPE_INT8) == 128 * 3 * 2048 * 768
    # INT8 projections are padded to 32 x 32 tiles
    assert lib.hm_packed_layer_bytes(3, 40, 70, capi.HM_DTYPE_INT8) == 3 * 3 * 64 * 96
    assert lib.hm_packed_layer_bytes(64, 2048, 768, capi.HM_DTYPE_FP32) == 64 * 3 * 2048 * 768 * 4
    layer = capi.HmLayer(128, 2048, 768, capi.HM_DTYPE_INT8, 1, 1, 1)
    a = lib.hm_moe_block_workspace_bytes(C.byref(layer), 4096, 8, 2, 3, 0)
    b = lib.hm_moe_block_workspace_bytes(C.byref(layer), 4096, 8, 2, 3, capi.HM_EXEC_GENERIC)
    # both paths hold the same buffers (z [P x I] floats, then its digits)
    assert a > 0 and a == b
    c = lib.hm_moe_block_workspace_bytes(C.byref(layer), 4096, 8, 2, 2, 0)
    assert a - c == 4096 * 8 * 768 + 4096 * 8 * 4, "one more Z digit plane and its digit sums"
    assert lib.hm_moe_block_workspace_bytes(C.byref(layer), 0, 8, 2, 2, 0) == 0
    # logits, then 4 K ranges of FP64 partials and norms, then W transposed
    assert lib.hm_route_workspace_bytes(4096, 2048, 128) == (
        4096 * 128 * 4 + 4 * (4096 * 128 + 4096 + 128) * 8 + 128 * 2048 * 4)
    assert lib.hm_route_workspace_bytes(100, 2048, 96) == (100 * 96 * 4 + 255) // 256 * 256


def test_argument_validation_without_device():
    """Invalid arguments are rejected before any device work (the reference's
    std::invalid_argument cases)."""
    st = capi.status
    assert st("hm_rmsnorm", 1, 1, 1, 4, 8, 0.0, None) == capi.HM_ERR_INVALID   # eps <= 0
    assert st("hm_router_topk", 1, 1, 4, 8, 3, 4, 3, 1, 1, None, None, 1, None) == capi.HM_ERR_INVALID
    assert st("hm_matmul_w8a32", 1, 2, 0.0, 0, 3, 1, 1, 1, 0, None, 0, None) == capi.HM_ERR_INVALID
    assert st("hm_matmul_w8a32", 1, 2, 1.0, 200, 3, 1, 1, 1, 0, None, 0, None) == capi.HM_ERR_INVALID
    assert st("hm_matmul_w8a32", 1, 2, 1.0, 0, 1, 1, 1, 1, 0, None, 0, None) == capi.HM_ERR_INVALID
    layer = capi.HmLayer(8, 64, 32, capi.HM_DTYPE_INT8, 1, 1, 1)
    io = capi.HmBlockIO()
    assert st("hm_moe_block_forward", C.byref(layer), 1, 1, 4, 9, 3, 2, 2, C.byref(io), 1, 10,
              None) == capi.HM_ERR_INVALID  # top_k > experts / no output
