"""ctypes wrapper of the CPU oracle (hm_oracle.c) and of the compiled
reference (oracle/_ref/libhm_ref.so, built only where /root/reference is
mounted).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product never imports this module.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "libhm_oracle.so"
REF_SO = HERE / "_ref" / "libhm_ref.so"

vp, i32, i64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float


class HmoLayer(C.Structure):
    _fields_ = [("experts", i64), ("hidden", i64), ("intermediate", i64), ("is_int8", i32),
                ("payload", vp), ("scale", vp), ("zero_point", vp)]


_ORACLE = None
_REF = None


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def oracle() -> C.CDLL:
    global _ORACLE
    if _ORACLE is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"{ORACLE_SO} is not built (make -C oracle)")
        lib = C.CDLL(str(ORACLE_SO))
        sig = {
            "hmo_rmsnorm": [vp, vp, vp, i64, i64, f32],
            "hmo_router_logits": [vp, vp, i64, i64, i64, vp],
            "hmo_route": [vp, vp, i64, i64, i64, i32, i32, i32, vp, vp],
            "hmo_group": [vp, vp, i64, i32, i64, vp, vp, vp, vp, vp],
            "hmo_matmul_w8a32": [vp, vp, f32, i32, vp, i64, i64, i64],
            "hmo_quantize_int8": [vp, i64, vp, vp, vp, vp],
            "hmo_expert_mlp": [C.POINTER(HmoLayer), i64, vp, i64, vp],
            "hmo_moe_block": [C.POINTER(HmoLayer), vp, vp, i64, i32, i32, i32, vp, vp, vp],
            "hmo_combine": [vp, vp, vp, vp, i64, i64, i64, vp],
            "hmo_limb_quantize": [vp, i64, i64, i64, i32, vp, vp],
            "hmo_limb_partials": [vp, i64, i64, i32, vp, i32, i64, vp],
            "hmo_limb_matmul": [vp, i64, i64, vp, f32, i32, i64, i32, vp],
            "hmo_limb_expert_mlp": [C.POINTER(HmoLayer), i64, vp, i64, i32, i32, vp],
            "hmo_moe_block_limbs": [C.POINTER(HmoLayer), vp, vp, i64, i32, i32, i32, i32, i32,
                                    vp, vp, vp],
        }
        for name, args in sig.items():
            getattr(lib, name).restype = C.c_int
            getattr(lib, name).argtypes = args
        for name in ("hmo_matmul_f32",):
            getattr(lib, name).restype = None
            getattr(lib, name).argtypes = [vp, vp, vp, i64, i64, i64]
        for name in ("hmo_silu",):
            getattr(lib, name).restype = None
            getattr(lib, name).argtypes = [vp, vp, i64]
        for name in ("hmo_mul", "hmo_add"):
            getattr(lib, name).restype = None
            getattr(lib, name).argtypes = [vp, vp, vp, i64]
        _ORACLE = lib
    return _ORACLE


def ref_available() -> bool:
    return REF_SO.exists()


def ref() -> C.CDLL:
    global _REF
    if _REF is None:
        if not REF_SO.exists():
            raise RuntimeError(f"{REF_SO} is not built (make -C oracle ref)")
        lib = C.CDLL(str(REF_SO))
        sig = {
            "hmref_rmsnorm": [vp, vp, vp, i64, i64, f32],
            "hmref_route_batch": [vp, vp, i64, i64, i64, i32, i32, i32, vp, vp, vp, vp, vp],
            "hmref_matmul_f32": [vp, vp, vp, i64, i64, i64],
            "hmref_matmul_w8a32": [vp, vp, f32, i32, vp, i64, i64, i64],
            "hmref_silu": [vp, vp, i64],
            "hmref_quantize_int8": [vp, i64, vp, vp, vp, vp],
            "hmref_plan_int8_gemm": [i64, i64, i64, i32, vp],
            "hmref_moe_block": [vp, i32, vp, vp, i64, i64, i64, vp, vp, i64, i32, i32, i32, vp,
                                vp, vp, vp, vp],
        }
        for name, args in sig.items():
            getattr(lib, name).restype = C.c_int
            getattr(lib, name).argtypes = args
        _REF = lib
    return _REF


def _check(rc: int, name: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{name} returned {rc}")


def f32a(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- oracle ----
def rmsnorm(x, gamma, eps=1e-6):
    x, gamma = f32a(x), f32a(gamma)
    y = np.empty_like(x)
    _check(oracle().hmo_rmsnorm(_p(x), _p(gamma), _p(y), x.shape[0], x.shape[1], eps), "hmo_rmsnorm")
    return y


def router_logits(h, w):
    h, w = f32a(h), f32a(w)
    out = np.empty((h.shape[0], w.shape[1]), np.float32)
    rc = oracle().hmo_router_logits(_p(h), _p(w), h.shape[0], h.shape[1], w.shape[1], _p(out))
    return rc, out


def route(h, w, k, softmax=True, renorm=True):
    h, w = f32a(h), f32a(w)
    T = h.shape[0]
    ids = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    rc = oracle().hmo_route(_p(h), _p(w), T, h.shape[1], w.shape[1], k, int(softmax),
                            int(renorm), _p(ids), _p(scores))
    return rc, ids, scores


def group(ids, scores, experts):
    ids = np.ascontiguousarray(ids, np.uint32)
    scores = f32a(scores)
    T, k = ids.shape
    counts = np.empty(experts, np.int32)
    offsets = np.empty(experts + 1, np.int32)
    ptok = np.empty(T * k, np.int32)
    pw = np.empty(T * k, np.float32)
    slots = np.empty(T * k, np.int32)
    _check(oracle().hmo_group(_p(ids), _p(scores), T, k, experts, _p(counts), _p(offsets),
                              _p(ptok), _p(pw), _p(slots)), "hmo_group")
    return counts, offsets, ptok, pw, slots.reshape(T, k)


def matmul_f32(x, w):
    x, w = f32a(x), f32a(w)
    y = np.empty((x.shape[0], w.shape[1]), np.float32)
    oracle().hmo_matmul_f32(_p(x), _p(w), _p(y), x.shape[0], x.shape[1], w.shape[1])
    return y


def matmul_w8a32(x, q, scale, zp):
    x, q = f32a(x), np.ascontiguousarray(q, np.int8)
    y = np.empty((x.shape[0], q.shape[1]), np.float32)
    _check(oracle().hmo_matmul_w8a32(_p(x), _p(q), scale, zp, _p(y), x.shape[0], x.shape[1],
                                     q.shape[1]), "hmo_matmul_w8a32")
    return y


def silu(x):
    x = f32a(x)
    y = np.empty_like(x)
    oracle().hmo_silu(_p(x), _p(y), x.size)
    return y


def quantize_int8(w):
    w = f32a(w)
    q = np.empty(w.shape, np.int8)
    s, z, e = f32(), i32(), f32()
    _check(oracle().hmo_quantize_int8(_p(w), w.size, _p(q), C.byref(s), C.byref(z), C.byref(e)),
           "hmo_quantize_int8")
    return q, s.value, z.value, e.value


def make_layer(payload, scale, zp):
    """payload [E, 3, H*I] (int8 or float32) in the reference layout."""
    E = payload.shape[0]
    return payload, scale, zp, E


def _layer_struct(payload, scale, zp, hidden, inter):
    is_int8 = payload.dtype == np.int8
    return HmoLayer(payload.shape[0], hidden, inter, int(is_int8), _p(payload),
                    _p(scale) if is_int8 else None, _p(zp) if is_int8 else None)


def expert_mlp(payload, scale, zp, expert, x, inter):
    """ExpertMlpExecutor::execute for one expert on gathered rows x [n x H]."""
    x = f32a(x)
    n, H = x.shape
    L = _layer_struct(payload, scale, zp, H, inter)
    y = np.empty((n, H), np.float32)
    _check(oracle().hmo_expert_mlp(C.byref(L), expert, _p(x), n, _p(y)), "hmo_expert_mlp")
    return y


def moe_block(payload, scale, zp, hidden, router_w, k, inter, softmax=True, renorm=True):
    hidden, router_w = f32a(hidden), f32a(router_w)
    T, H = hidden.shape
    L = _layer_struct(payload, scale, zp, H, inter)
    out = np.empty((T, H), np.float32)
    ids = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    _check(oracle().hmo_moe_block(C.byref(L), _p(hidden), _p(router_w), T, k, int(softmax),
                                  int(renorm), _p(out), _p(ids), _p(scores)), "hmo_moe_block")
    return out, ids, scores


def moe_block_limbs(payload, scale, zp, hidden, router_w, k, inter, limbs_x, limbs_z,
                    softmax=True, renorm=True):
    hidden, router_w = f32a(hidden), f32a(router_w)
    T, H = hidden.shape
    L = _layer_struct(payload, scale, zp, H, inter)
    out = np.empty((T, H), np.float32)
    ids = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    _check(oracle().hmo_moe_block_limbs(C.byref(L), _p(hidden), _p(router_w), T, k, int(softmax),
                                        int(renorm), limbs_x, limbs_z, _p(out), _p(ids),
                                        _p(scores)), "hmo_moe_block_limbs")
    return out, ids, scores


def limb_quantize(x, limbs):
    x = f32a(x)
    rows, n = x.shape
    digits = np.empty((limbs, rows, n), np.int8)
    scales = np.empty(rows, np.float32)
    _check(oracle().hmo_limb_quantize(_p(x), rows, n, n, limbs, _p(digits), _p(scales)),
           "hmo_limb_quantize")
    return digits, scales


def limb_partials(digits, q, zp):
    digits = np.ascontiguousarray(digits, np.int8)
    q = np.ascontiguousarray(q, np.int8)
    limbs, rows, inner = digits.shape
    out = np.empty((limbs, rows, q.shape[1]), np.int32)
    _check(oracle().hmo_limb_partials(_p(digits), rows, inner, limbs, _p(q), zp, q.shape[1],
                                      _p(out)), "hmo_limb_partials")
    return out


def limb_matmul(x, q, scale, zp, limbs):
    x, q = f32a(x), np.ascontiguousarray(q, np.int8)
    y = np.empty((x.shape[0], q.shape[1]), np.float32)
    _check(oracle().hmo_limb_matmul(_p(x), x.shape[0], x.shape[1], _p(q), scale, zp, q.shape[1],
                                    limbs, _p(y)), "hmo_limb_matmul")
    return y


def combine(y_grouped, offsets, perm_tokens, perm_weights, tokens):
    y_grouped = f32a(y_grouped)
    E = len(offsets) - 1
    out = np.empty((tokens, y_grouped.shape[1]), np.float32)
    _check(oracle().hmo_combine(_p(y_grouped), _p(np.ascontiguousarray(offsets, np.int32)),
                                _p(np.ascontiguousarray(perm_tokens, np.int32)),
                                _p(f32a(perm_weights)), E, tokens, y_grouped.shape[1], _p(out)),
           "hmo_combine")
    return out


# ------------------------------------------------------------- reference ----
def ref_rmsnorm(x, gamma, eps=1e-6):
    x, gamma = f32a(x), f32a(gamma)
    y = np.empty_like(x)
    _check(ref().hmref_rmsnorm(_p(x), _p(gamma), _p(y), x.shape[0], x.shape[1], eps), "hmref_rmsnorm")
    return y


def ref_route_batch(h, w, k, softmax=True, renorm=True):
    h, w = f32a(h), f32a(w)
    T, E = h.shape[0], w.shape[1]
    ids = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    counts = np.empty(E, np.int32)
    ptok = np.empty(T * k, np.int32)
    pw = np.empty(T * k, np.float32)
    rc = ref().hmref_route_batch(_p(h), _p(w), T, h.shape[1], E, k, int(softmax), int(renorm),
                                 _p(ids), _p(scores), _p(counts), _p(ptok), _p(pw))
    return rc, ids, scores, counts, ptok, pw


def ref_matmul_f32(x, w):
    x, w = f32a(x), f32a(w)
    y = np.empty((x.shape[0], w.shape[1]), np.float32)
    _check(ref().hmref_matmul_f32(_p(x), _p(w), _p(y), x.shape[0], x.shape[1], w.shape[1]),
           "hmref_matmul_f32")
    return y


def ref_matmul_w8a32(x, q, scale, zp):
    x, q = f32a(x), np.ascontiguousarray(q, np.int8)
    y = np.empty((x.shape[0], q.shape[1]), np.float32)
    _check(ref().hmref_matmul_w8a32(_p(x), _p(q), scale, zp, _p(y), x.shape[0], x.shape[1],
                                    q.shape[1]), "hmref_matmul_w8a32")
    return y


def ref_silu(x):
    x = f32a(x)
    y = np.empty_like(x)
    _check(ref().hmref_silu(_p(x), _p(y), x.size), "hmref_silu")
    return y


def ref_quantize_int8(w):
    w = f32a(w)
    q = np.empty(w.shape, np.int8)
    s, z, e = f32(), i32(), f32()
    _check(ref().hmref_quantize_int8(_p(w), w.size, _p(q), C.byref(s), C.byref(z), C.byref(e)),
           "hmref_quantize_int8")
    return q, s.value, z.value, e.value


def ref_plan_int8_gemm(rows, inner, cols, mode=0):
    out = np.empty(4, np.int64)
    rc = ref().hmref_plan_int8_gemm(rows, inner, cols, mode, _p(out))
    return rc, out


def ref_moe_block(payload, scale, zp, hidden, router_w, k, inter, softmax=True, renorm=True,
                  expert_out=False):
    hidden, router_w = f32a(hidden), f32a(router_w)
    T, H = hidden.shape
    E = payload.shape[0]
    is_int8 = payload.dtype == np.int8
    out = np.empty((T, H), np.float32)
    ids = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    counts = np.empty(E, np.int32)
    yo = np.empty((T * k, H), np.float32) if expert_out else None
    _check(ref().hmref_moe_block(_p(payload), int(is_int8), _p(scale) if is_int8 else None,
                                 _p(zp) if is_int8 else None, E, H, inter, _p(hidden),
                                 _p(router_w), T, k, int(softmax), int(renorm), _p(out), _p(ids),
                                 _p(scores), _p(counts), _p(yo)), "hmref_moe_block")
    return out, ids, scores, counts, yo
