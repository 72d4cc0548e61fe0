#!/usr/bin/env python3
"""Writes the golden vectors in tests/golden/ from the compiled reference.

Runs only in the container where /root/reference is mounted: it needs
oracle/_ref/libhm_ref.so (make -C oracle ref), i.e. the reference's own CPU
sources (router, tensor backend, quantiser, RMSNorm, expert executor and
MoERuntime::executeBatch over an on-disk ExpertStore) driven by
oracle/ref_driver.cpp.  Inputs are regenerated from seeds with the build's
IEEE-only generator (hypermoe-engine_amd/host/hm_synth.c); each fixture stores
a SHA-256 of its inputs so a changed generator is caught, and the reference's
outputs.  Fixtures are data only (.npz, no pickles).

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO / "hypermoe-engine_amd"))
sys.path.insert(0, str(REPO / "oracle"))

import hm_oracle as O  # noqa: E402
from hmoe import synth  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def block_inputs(name, seed, T, H, E, I, int8, skew=False):
    payload, scale, zp = synth.expert_layer(seed, 0, E, H, I, int8)
    raw = synth.raw_hidden(seed, T, H)
    h = O.ref_rmsnorm(raw, np.ones(H, np.float32), 1e-6)
    w = synth.router_weights(seed, 0, H, E)
    if skew:
        synth.apply_skew(h, w, synth.zipf_bias(seed, E))
    return payload, scale, zp, raw, h, w


def make_block(name, seed, T, H, E, I, k, int8, skew=False):
    payload, scale, zp, raw, h, w = block_inputs(name, seed, T, H, E, I, int8, skew)
    out, ids, scores, counts, yo = O.ref_moe_block(payload, scale, zp, h, w, k, I,
                                                   expert_out=T * k * H <= 4096)
    rec = dict(seed=seed, T=T, H=H, E=E, I=I, k=k, int8=int(int8), skew=int(skew),
               input_sha=sha(payload, scale, zp, raw, w), hidden_sha=sha(h), out=out, ids=ids,
               scores=scores, counts=counts)
    if yo is not None:
        rec["expert_out"] = yo
    np.savez_compressed(HERE / f"{name}.npz", **rec)
    print(f"{name}: T={T} E={E} int8={int8} out max {np.abs(out).max():.4g}")


def make_ops():
    rng = np.random.default_rng(20240601)
    rec = {}
    # RMSNorm (RMSNorm.cpp:65-77) on rows of varied magnitude
    x = (rng.standard_normal((8, 2048)) * rng.uniform(1e-3, 1e3, (8, 1))).astype(np.float32)
    g = rng.uniform(0.5, 2.0, 2048).astype(np.float32)
    rec["rms_x"], rec["rms_g"], rec["rms_y"] = x, g, O.ref_rmsnorm(x, g, 1e-6)
    # SiLU (Activation.cpp:44) on a wide grid
    s = np.concatenate([np.linspace(-100, 100, 20001, dtype=np.float32),
                        (rng.standard_normal(20000) * 5).astype(np.float32)])
    rec["silu_x"], rec["silu_y"] = s, O.ref_silu(s)
    # INT8 packer (Quantization.cpp:45-79)
    wq = (0.02 * rng.standard_normal(4096)).astype(np.float32)
    wq[::97] = 0.0
    q, sc, z, err = O.ref_quantize_int8(wq)
    rec["q_w"], rec["q_q"], rec["q_meta"] = wq, q, np.array([sc, z, err], np.float64)
    # W8A32 GEMM (CpuTensorBackend.cpp:173-186) on the phase23 inputs
    for (r, kk, c) in [(1, 257, 65), (2, 513, 33), (3, 129, 7), (1, 2048, 64)]:
        i = np.arange(r * kk)
        xa = (((i % 29) - 14).astype(np.float32) / np.float32(29.0)).reshape(r, kk)
        j = np.arange(kk * c)
        qa = (((j * 13) % 255) - 127).astype(np.int8).reshape(kk, c)
        rec[f"w8_{r}_{kk}_{c}"] = O.ref_matmul_w8a32(xa, qa, 0.003, -3)
    # FP32 GEMM (CpuTensorBackend.cpp:120-129)
    a = rng.standard_normal((5, 300)).astype(np.float32)
    b = rng.standard_normal((300, 17)).astype(np.float32)
    rec["f32_a"], rec["f32_b"], rec["f32_y"] = a, b, O.ref_matmul_f32(a, b)
    # router with and without softmax / renorm, plus ties
    h = rng.standard_normal((24, 96)).astype(np.float32)
    w = (0.05 * rng.standard_normal((96, 40))).astype(np.float32)
    w[:, 20:] = w[:, :20]  # duplicated columns -> exact ties
    rec["rt_h"], rec["rt_w"] = h, w
    for sm, rn in ((1, 1), (1, 0), (0, 0)):
        rc, ids, scores, counts, ptok, pw = O.ref_route_batch(h, w, 6, sm, rn)
        assert rc == 0
        rec[f"rt_{sm}{rn}_ids"], rec[f"rt_{sm}{rn}_scores"] = ids, scores
        rec[f"rt_{sm}{rn}_counts"], rec[f"rt_{sm}{rn}_ptok"] = counts, ptok
        rec[f"rt_{sm}{rn}_pw"] = pw
    # launch plans (Int8GemmPlan.cpp:29-53)
    plans = []
    for dims in [(1, 2048, 768), (1, 768, 2048), (1, 8, 8), (2, 257, 65), (1, 8193, 65),
                 (4, 4096, 128), (1, 511, 64)]:
        for mode in (0, 1, 2):
            rc, out = O.ref_plan_int8_gemm(*dims, mode)
            plans.append([*dims, mode, rc, *out.tolist()])
    rec["plans"] = np.array(plans, np.int64)
    np.savez_compressed(HERE / "ops.npz", **rec)
    print("ops: written")


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libhm_ref.so is not built; run make -C oracle ref (needs /root/reference)")
    make_ops()
    make_block("block_tiny_fp32", 7, 12, 64, 8, 32, 2, False)
    make_block("block_tiny_int8", 7, 12, 64, 8, 32, 2, True)
    make_block("block_c1_fp32", 20240601, 16, 2048, 64, 768, 8, False)
    for T in (1, 4, 16):
        make_block(f"block_c3_{T}_int8", 20240601, T, 2048, 128, 768, 8, True)
    make_block("block_c4slice_int8", 20240601, 24, 2048, 128, 768, 8, True, skew=True)


if __name__ == "__main__":
    main()
