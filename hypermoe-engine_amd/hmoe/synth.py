"""Seeded synthetic inputs (binding of host/hm_synth.c; the generator is
specified in that file's header) and the benchmark configurations.

Configurations (BASELINE.json `configs`):
  C1  FP32 experts, T=16,   H=2048, E=64,  k=8, I=768 (reference CPU case)
  C2  FP32 experts, T=512,  otherwise C1
  C3  INT8 experts, T in {1, 4, 16}, H=2048, E=128, k=8, I=768 (decode)
  C4  INT8 experts, T=4096, E=128, k=8, Zipf(s=1.1)-skewed routing (prefill)
  C5  48 layers of the C3/C4 block with RMSNorm and residual (stack)

Hidden states are N(0,1) passed through RMSNorm (eps 1e-6, unit gamma);
router and expert weights are N(0, 0.02); INT8 experts are packed per
projection with the reference packer (Quantization.cpp:45-79).

Skewed routing (C4) is encoded so the unmodified reference router can route
it: feature H-1 of every post-norm hidden row is set to 1.0 and router row
H-1 holds a per-expert bias b_e = beta * ln(zipf_e), zipf_e = rank_e^-1.1
with the ranks a seeded permutation of the experts.  beta = 0.9 puts about
10x the mean load on the hottest expert at T=4096.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from . import build as _build

TAG_HIDDEN = 1


def tag_router(layer: int) -> int:
    return 0x100 + layer


def tag_expert(layer: int, expert: int, proj: int) -> int:
    return (1 << 40) | (layer << 20) | (expert << 4) | proj


_LIB: C.CDLL | None = None


def load() -> C.CDLL:
    global _LIB
    if _LIB is None:
        path = _build.SYNTH_SO
        if not path.exists():
            raise RuntimeError(f"{path} is not built: run __graft_entry__.build()")
        lib = C.CDLL(str(path))
        lib.hm_synth_key.restype = C.c_uint64
        lib.hm_synth_key.argtypes = [C.c_uint64, C.c_uint64]
        lib.hm_synth_u64.restype = C.c_uint64
        lib.hm_synth_u64.argtypes = [C.c_uint64, C.c_uint64]
        lib.hm_synth_ln.restype = C.c_double
        lib.hm_synth_ln.argtypes = [C.c_double]
        lib.hm_synth_cossin.restype = None
        lib.hm_synth_cossin.argtypes = [C.c_double, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        lib.hm_synth_normal.restype = None
        lib.hm_synth_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_float,
                                        C.c_float, C.c_void_p]
        lib.hm_synth_layer.restype = C.c_int
        lib.hm_synth_layer.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_int64,
                                       C.c_int64, C.c_float, C.c_int, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_int]
        _LIB = lib
    return _LIB


def normal(seed: int, tag: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().hm_synth_normal(seed, tag, n, mean, std, out.ctypes.data)
    return out


def expert_layer(seed: int, layer: int, experts: int, hidden: int, inter: int,
                 int8: bool, std: float = 0.02, threads: int = 8):
    """Reference payload layout: [E, 3, H*I] (gate [HxI], up [HxI], down [IxH])."""
    dtype = np.int8 if int8 else np.float32
    payload = np.empty((experts, 3, hidden * inter), dtype=dtype)
    scale = np.empty((experts, 3), dtype=np.float32)
    zp = np.empty((experts, 3), dtype=np.int32)
    rc = load().hm_synth_layer(seed, layer, experts, hidden, inter, std, int(int8),
                               payload.ctypes.data, scale.ctypes.data, zp.ctypes.data, threads)
    if rc:
        raise RuntimeError("hm_synth_layer failed")
    if not int8:
        scale[:] = 1.0
        zp[:] = 0
    return payload, scale, zp


def router_weights(seed: int, layer: int, hidden: int, experts: int) -> np.ndarray:
    return normal(seed, tag_router(layer), hidden * experts, 0.0, 0.02).reshape(hidden, experts)


def raw_hidden(seed: int, tokens: int, hidden: int) -> np.ndarray:
    return normal(seed, TAG_HIDDEN, tokens * hidden).reshape(tokens, hidden)


def zipf_bias(seed: int, experts: int, s: float = 1.1, beta: float = 0.43) -> np.ndarray:
    """b_e = beta * ln(rank_e^-s), ranks a seeded permutation of 1..E.

    A Zipf(s) popularity ranking expressed as a logit offset.  beta sets the
    strength: at C4 (4096 tokens, 128 experts, top-8, post-RMSNorm hidden,
    N(0, 0.02) router) beta = 0.43 gives the hottest expert 10.0x the mean
    load (2559 of 32768 assignments), every expert at least 48."""
    key = load().hm_synth_key(seed, 0x5A1F)
    u = [load().hm_synth_u64(key, i) for i in range(experts)]
    order = sorted(range(experts), key=lambda e: (u[e], e))
    ranks = np.empty(experts, dtype=np.float64)
    for r, e in enumerate(order):
        ranks[e] = r + 1
    return (beta * (-s) * np.log(ranks)).astype(np.float32)


def apply_skew(hidden_post_norm: np.ndarray, router_w: np.ndarray, bias: np.ndarray) -> None:
    """Encode a per-expert logit bias through feature H-1 (in place)."""
    hidden_post_norm[:, -1] = 1.0
    router_w[-1, :] = bias


@dataclass(frozen=True)
class Config:
    name: str
    tokens: int
    hidden: int = 2048
    experts: int = 128
    top_k: int = 8
    inter: int = 768
    int8: bool = True
    skew: bool = False
    layers: int = 1
    seed: int = 20240601


CONFIGS = {
    "C1": Config("C1", tokens=16, experts=64, int8=False),
    "C2": Config("C2", tokens=512, experts=64, int8=False),
    "C3-1": Config("C3-1", tokens=1),
    "C3-4": Config("C3-4", tokens=4),
    "C3-16": Config("C3-16", tokens=16),
    "C4": Config("C4", tokens=4096, skew=True),
    # not a BASELINE config: a mid-size INT8 prefill (16 rows per expert on
    # average), where most groups are skinny (the split-K comparison)
    "M256": Config("M256", tokens=256, skew=True),
    "C5": Config("C5", tokens=2048, layers=48),
}


def algorithmic_bytes(cfg: Config, unique_experts: int) -> int:
    """B = U*3*H*I*s_w + H*E*4 + 2*T*H*4 (weights touched, router, in/out)."""
    sw = 1 if cfg.int8 else 4
    return (unique_experts * 3 * cfg.hidden * cfg.inter * sw
            + cfg.hidden * cfg.experts * 4 + 2 * cfg.tokens * cfg.hidden * 4)


def algorithmic_ops(cfg: Config) -> int:
    """F = 2*T*k*3*H*I (multiply-adds counted as 2)."""
    return 2 * cfg.tokens * cfg.top_k * 3 * cfg.hidden * cfg.inter


def spec_u64(key: int, index: int) -> int:
    """Pure-Python SplitMix64 stream (spec check of the C generator)."""
    m = (1 << 64) - 1
    z = (key + (index + 1) * 0x9E3779B97F4A7C15) & m
    z ^= z >> 30
    z = (z * 0xBF58476D1CE4E5B9) & m
    z ^= z >> 27
    z = (z * 0x94D049BB133111EB) & m
    z ^= z >> 31
    return z


def spec_mix(z: int) -> int:
    m = (1 << 64) - 1
    z &= m
    z ^= z >> 30
    z = (z * 0xBF58476D1CE4E5B9) & m
    z ^= z >> 27
    z = (z * 0x94D049BB133111EB) & m
    z ^= z >> 31
    return z


def spec_key(seed: int, tag: int) -> int:
    return spec_mix((seed + spec_mix(tag)) & ((1 << 64) - 1))


def spec_normal_pair(seed: int, tag: int, j: int, mean: float, std: float):
    """Pure-Python restatement of one Box-Muller pair, using math.log/cos
    (accuracy check; the C generator uses its own series)."""
    key = spec_key(seed, tag)
    a, b = spec_u64(key, 2 * j), spec_u64(key, 2 * j + 1)
    u1 = ((a >> 11) + 1) * 2.0 ** -53
    u2 = (b >> 11) * 2.0 ** -53
    r = math.sqrt(-2.0 * math.log(u1))
    return mean + std * r * math.cos(2 * math.pi * u2), mean + std * r * math.sin(2 * math.pi * u2)
