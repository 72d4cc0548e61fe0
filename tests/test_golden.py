"""The oracle against golden vectors written by the compiled reference
(tests/golden/make_golden.py): bit-exact.  CPU only."""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact
from hmoe import synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


BLOCKS = ["block_tiny_fp32", "block_tiny_int8", "block_c1_fp32", "block_c3_1_int8",
          "block_c3_4_int8", "block_c3_16_int8", "block_c4slice_int8"]


@pytest.mark.parametrize("name", BLOCKS)
def test_moe_block_golden(name):
    """MoERuntime::executeBatch CPU path (core/runtime/MoERuntime.cpp:58-349)
    as run by the compiled reference, against the oracle restatement."""
    g = load(name)
    seed, T, H, E, I, k = (int(g[x]) for x in ("seed", "T", "H", "E", "I", "k"))
    int8, skew = bool(g["int8"]), bool(g["skew"])
    payload, scale, zp = synth.expert_layer(seed, 0, E, H, I, int8)
    raw = synth.raw_hidden(seed, T, H)
    w = synth.router_weights(seed, 0, H, E)
    h = O.rmsnorm(raw, np.ones(H, np.float32), 1e-6)
    if skew:
        synth.apply_skew(h, w, synth.zipf_bias(seed, E))
    assert sha(payload, scale, zp, raw, w) == str(g["input_sha"]), "input generator drifted"
    assert sha(h) == str(g["hidden_sha"]), "oracle RMSNorm differs from the reference's"
    out, ids, scores = O.moe_block(payload, scale, zp, h, w, k, I)
    assert_bitexact(ids, g["ids"], "ids")
    assert_bitexact(scores, g["scores"], "scores")
    assert_bitexact(out, g["out"], "block output")
    counts, *_ = O.group(ids, scores, E)
    assert_bitexact(counts, g["counts"], "group sizes")
    if "expert_out" in g.files:
        # per-group expert outputs (BatchLayerExecutionResult::expertOutputs)
        counts, offsets, ptok, pw, _ = O.group(ids, scores, E)
        rows = []
        for e in range(E):
            if counts[e]:
                xg = h[ptok[offsets[e]:offsets[e + 1]]]
                rows.append(_expert(payload, scale, zp, e, xg, H, I))
        assert_bitexact(np.concatenate(rows), g["expert_out"], "expert outputs")


def _expert(payload, scale, zp, e, x, H, I):
    x = np.ascontiguousarray(x, np.float32)
    is_int8 = payload.dtype == np.int8
    base = payload[e]
    gate = base[0].reshape(H, I)
    up = base[1].reshape(H, I)
    down = base[2].reshape(I, H)
    if is_int8:
        g = O.matmul_w8a32(x, gate, scale[e, 0], zp[e, 0])
        u = O.matmul_w8a32(x, up, scale[e, 1], zp[e, 1])
        z = O.silu(g) * u
        return O.matmul_w8a32(z, down, scale[e, 2], zp[e, 2])
    g = O.matmul_f32(x, gate)
    u = O.matmul_f32(x, up)
    return O.matmul_f32(O.silu(g) * u, down)


def test_ops_golden():
    g = load("ops")
    assert_bitexact(O.rmsnorm(g["rms_x"], g["rms_g"], 1e-6), g["rms_y"], "rmsnorm")
    assert_bitexact(O.silu(g["silu_x"]), g["silu_y"], "silu")
    q, s, z, err = O.quantize_int8(g["q_w"])
    assert_bitexact(q, g["q_q"], "quantized bytes")
    assert (np.float32(s), z, np.float32(err)) == tuple(
        np.array(g["q_meta"][:1], np.float32).tolist() + [int(g["q_meta"][1])]
        + np.array(g["q_meta"][2:], np.float32).tolist())
    for (r, kk, c) in [(1, 257, 65), (2, 513, 33), (3, 129, 7), (1, 2048, 64)]:
        i = np.arange(r * kk)
        xa = (((i % 29) - 14).astype(np.float32) / np.float32(29.0)).reshape(r, kk)
        j = np.arange(kk * c)
        qa = (((j * 13) % 255) - 127).astype(np.int8).reshape(kk, c)
        assert_bitexact(O.matmul_w8a32(xa, qa, 0.003, -3), g[f"w8_{r}_{kk}_{c}"], "w8a32")
    assert_bitexact(O.matmul_f32(g["f32_a"], g["f32_b"]), g["f32_y"], "fp32 gemm")
    for sm, rn in ((1, 1), (1, 0), (0, 0)):
        rc, ids, scores = O.route(g["rt_h"], g["rt_w"], 6, sm, rn)
        assert rc == 0
        assert_bitexact(ids, g[f"rt_{sm}{rn}_ids"], "router ids")
        assert_bitexact(scores, g[f"rt_{sm}{rn}_scores"], "router scores")
        counts, offsets, ptok, pw, _ = O.group(ids, scores, 40)
        assert_bitexact(counts, g[f"rt_{sm}{rn}_counts"], "counts")
        assert_bitexact(ptok, g[f"rt_{sm}{rn}_ptok"], "permutation")
        assert_bitexact(pw, g[f"rt_{sm}{rn}_pw"], "permuted weights")


def test_plan_golden():
    """hm_plan_int8_gemm keeps the reference's launch-plan decisions
    (Int8GemmPlan.cpp:29-53): mode, partitions and scratch; the workgroup
    count is this build's own (64 columns per workgroup)."""
    import ctypes as C
    from hmoe import capi
    for row in load("ops")["plans"]:
        rows, inner, cols, mode, rc, impl, parts, blocks, scratch = (int(v) for v in row)
        plan = capi.HmInt8GemmPlan()
        mine = capi.status("hm_plan_int8_gemm", rows, inner, cols, mode, C.byref(plan))
        assert (mine == 0) == (rc == 0)
        if rc != 0:
            continue
        assert plan.implementation == impl  # Int8GemmMode: 1 Reference, 2 Cooperative
        assert plan.partitions == parts and plan.scratch_elements == scratch
        if impl == 1:
            assert plan.blocks == blocks  # ceil(M*N/256), same as the reference
