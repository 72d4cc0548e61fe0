"""ctypes binding of the C ABI in include/hm_moe.h (libhm_kernels.so).

Loading fails loudly when the HIP library has not been built: there is no
CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

from . import build as _build

c_i32, c_i64, c_u32, c_f32, c_sz = C.c_int32, C.c_int64, C.c_uint32, C.c_float, C.c_size_t
vp = C.c_void_p

HM_OK, HM_ERR_INVALID, HM_ERR_OVERFLOW, HM_ERR_RUNTIME, HM_ERR_UNSUPPORTED = 0, 1, 2, 3, 4
HM_STATUS_NONFINITE_SCORE, HM_STATUS_SOFTMAX_FAILED, HM_STATUS_RENORM_FAILED = 1, 2, 4
HM_ROUTE_SOFTMAX, HM_ROUTE_RENORM, HM_EXEC_GENERIC, HM_EXEC_LIMBS = 1, 2, 0x100, 0x200
HM_EXEC_SPLIT_K = 0x800
HM_GEMV_MAX_TOKENS = 16
HM_GEMV_MAX_PAIRS = 64
HM_EXEC_ROUTE_SEQUENTIAL = 0x400
HM_DTYPE_FP32, HM_DTYPE_INT8 = 0, 3


class HmLayer(C.Structure):
    _fields_ = [("experts", c_i64), ("hidden", c_i64), ("intermediate", c_i64),
                ("dtype", c_i32), ("packed", vp), ("scale", vp), ("zero_point", vp)]


class HmBlockIO(C.Structure):
    _fields_ = [("out", vp), ("ids", vp), ("scores", vp), ("counts", vp), ("offsets", vp),
                ("perm_tokens", vp), ("perm_weights", vp), ("expert_out", vp),
                ("status", vp), ("residual", vp), ("events", C.POINTER(vp))]


HM_BLOCK_EVENTS = 7
HM_NOALLOC_WORKSPACE_BYTES = 64 << 20


class HmInt8GemmPlan(C.Structure):
    _fields_ = [("implementation", c_i32), ("partitions", c_i64), ("blocks", c_i64),
                ("scratch_elements", c_i64)]


# name -> (restype, argtypes); mirrors include/hm_moe.h
SIGNATURES = {
    "hm_abi_version": (c_i32, []),
    "hm_status_string": (C.c_char_p, [c_i32]),
    "hm_last_hip_error": (c_i32, []),
    "hm_device_count": (c_i32, [C.POINTER(C.c_int)]),
    "hm_set_device": (c_i32, [c_i32]),
    "hm_device_alloc": (c_i32, [C.POINTER(vp), c_sz]),
    "hm_device_free": (c_i32, [vp]),
    "hm_host_alloc": (c_i32, [C.POINTER(vp), c_sz]),
    "hm_host_free": (c_i32, [vp]),
    "hm_memcpy_h2d": (c_i32, [vp, vp, c_sz, vp]),
    "hm_memcpy_d2h": (c_i32, [vp, vp, c_sz, vp]),
    "hm_memcpy_d2d": (c_i32, [vp, vp, c_sz, vp]),
    "hm_stream_create": (c_i32, [C.POINTER(vp)]),
    "hm_stream_destroy": (c_i32, [vp]),
    "hm_stream_synchronize": (c_i32, [vp]),
    "hm_event_create": (c_i32, [C.POINTER(vp)]),
    "hm_event_destroy": (c_i32, [vp]),
    "hm_event_record": (c_i32, [vp, vp]),
    "hm_event_synchronize": (c_i32, [vp]),
    "hm_stream_wait_event": (c_i32, [vp, vp]),
    "hm_event_elapsed_ms": (c_i32, [C.POINTER(c_f32), vp, vp]),
    "hm_mem_info": (c_i32, [C.POINTER(c_sz), C.POINTER(c_sz)]),
    "hm_rmsnorm": (c_i32, [vp, vp, vp, c_i64, c_i64, c_f32, vp]),
    "hm_route_workspace_bytes": (c_sz, [c_i64, c_i64, c_i64]),
    "hm_router_topk": (c_i32, [vp, vp, c_i64, c_i64, c_i64, c_i32, c_u32, vp, vp, vp, vp, vp, vp]),
    "hm_permute_workspace_bytes": (c_sz, [c_i64, c_i32, c_i64]),
    "hm_permute": (c_i32, [vp, vp, c_i64, c_i32, c_i64, vp, vp, vp, vp, vp, vp, vp]),
    "hm_gather_rows": (c_i32, [vp, vp, c_i64, c_i64, vp, vp]),
    "hm_plan_int8_gemm": (c_i32, [c_i64, c_i64, c_i64, c_i32, C.POINTER(HmInt8GemmPlan)]),
    "hm_matmul_w8a32": (c_i32, [vp, vp, c_f32, c_i32, vp, c_i64, c_i64, c_i64, c_i32, vp, c_sz, vp]),
    "hm_matmul_f32": (c_i32, [vp, vp, vp, c_i64, c_i64, c_i64, vp]),
    "hm_silu": (c_i32, [vp, vp, c_i64, vp]),
    "hm_mul": (c_i32, [vp, vp, vp, c_i64, vp]),
    "hm_add": (c_i32, [vp, vp, vp, c_i64, vp]),
    "hm_combine": (c_i32, [vp, vp, vp, vp, c_i64, c_i32, c_i64, vp, vp, vp]),
    "hm_quantize_int8_host": (c_i32, [vp, c_i64, vp, vp, vp, vp]),
    "hm_packed_layer_bytes": (c_sz, [c_i64, c_i64, c_i64, c_i32]),
    "hm_pack_layer": (c_i32, [vp, c_i64, c_i64, c_i64, c_i32, vp, vp]),
    "hm_moe_block_workspace_bytes": (c_sz, [C.POINTER(HmLayer), c_i64, c_i32, c_i32, c_i32,
                                            c_u32]),
    "hm_moe_block_forward": (c_i32, [C.POINTER(HmLayer), vp, vp, c_i64, c_i32, c_u32, c_i32,
                                     c_i32, C.POINTER(HmBlockIO), vp, c_sz, vp]),
    "hm_moe_block_forward_noalloc": (c_i32, [C.POINTER(HmLayer), vp, vp, c_i64, c_i32, c_u32,
                                             c_i32, c_i32, C.POINTER(HmBlockIO), vp]),
    "hm_moe_layer_forward": (c_i32, [C.POINTER(HmLayer), vp, vp, c_f32, vp, vp, c_i64, c_i32,
                                     c_u32, c_i32, c_i32, C.POINTER(HmBlockIO), vp, c_sz, vp]),
    "hm_limb_quantize_rows": (c_i32, [vp, c_i64, c_i64, c_i32, vp, vp, vp]),
    "hm_limb_partials": (c_i32, [vp, c_i64, c_i64, c_i32, vp, c_i32, c_i64, vp, vp]),
    "hm_debug_expf": (c_i32, [vp, vp, c_i64, vp]),
}

_LIB: C.CDLL | None = None


class HmError(RuntimeError):
    def __init__(self, name: str, status: int, hip: int = 0):
        self.status = status
        self.hip_error = hip
        super().__init__(f"{name} failed: status {status}"
                         + (f" (hipError {hip})" if hip else ""))


def lib_path() -> Path:
    return _build.KERNELS_SO


def load() -> C.CDLL:
    """Load libhm_kernels.so; raises if it is missing (no fallback)."""
    global _LIB
    if _LIB is None:
        path = lib_path()
        if not path.exists():
            raise RuntimeError(f"{path} is not built: run __graft_entry__.build() "
                               "(the HIP extension is required; there is no CPU fallback)")
        lib = C.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def call(name: str, *args) -> int:
    """Call a C-ABI function and raise HmError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if SIGNATURES[name][0] is c_i32 and name not in ("hm_abi_version", "hm_last_hip_error") and rc != 0:
        raise HmError(name, rc, lib.hm_last_hip_error())
    return rc


def status(name: str, *args) -> int:
    """Call and return the raw status (for error-path tests)."""
    return getattr(load(), name)(*args)
