"""The oracle against the closed-form known answers held by the reference's
own tests, and against mathematics that fixes the result independently
(brute force, textbook algorithms, invariants).  CPU only.

Each check names the reference test it restates.  A deliberately wrong
oracle (dropped term, wrong sign, swapped operand) fails at least one."""
from __future__ import annotations

import itertools
import math

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact


def test_fp32_gemm_closed_form():
    """tests/phase5_tests.cpp:147-160."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert O.matmul_f32(a, b).tolist() == [[58, 64], [139, 154]]


def test_silu_values():
    """tests/phase6_tests.cpp:168-177 (SiLU of -2..2) and the definition
    x / (1 + e^-x) in double."""
    x = np.array([-2, -1, 0, 1, 2], np.float32)
    np.testing.assert_allclose(O.silu(x), [-0.23840584, -0.26894143, 0.0, 0.73105860,
                                            1.76159418], rtol=1e-6, atol=1e-7)
    xs = np.linspace(-30, 30, 10001, dtype=np.float32)
    exact = xs.astype(np.float64) / (1 + np.exp(-xs.astype(np.float64)))
    assert np.max(np.abs(O.silu(xs) - exact) / np.maximum(np.abs(exact), 1e-30)) < 4e-7


def test_gated_mlp_closed_form():
    """tests/phase6_tests.cpp:198-222: input [1,2], gate I, up diag(2,3),
    down [1, 0.5]^T -> silu(1)*2 + silu(2)*6*0.5, through the oracle's
    expert MLP (ExpertExecutor.cpp:97-131) with H = I = 2 (down padded with a
    zero output column)."""
    payload = np.zeros((1, 3, 4), np.float32)
    payload[0, 0] = [1, 0, 0, 1]      # gate [H x I]
    payload[0, 1] = [2, 0, 0, 3]      # up
    payload[0, 2] = [1, 0, 0.5, 0]    # down [I x H]
    x = np.array([[1.0, 2.0]], np.float32)
    L = O.HmoLayer(1, 2, 2, 0, payload.ctypes.data, None, None)
    y = np.empty((1, 2), np.float32)
    import ctypes
    assert O.oracle().hmo_expert_mlp(ctypes.byref(L), 0, x.ctypes.data, 1, y.ctypes.data) == 0
    silu = lambda v: v / (1 + math.exp(-v))  # noqa: E731
    expected = silu(1.0) * 2.0 + silu(2.0) * 6.0 * 0.5
    assert abs(float(y[0, 0]) - expected) < 1e-6 and y[0, 1] == 0.0


def test_router_closed_forms():
    """tests/phase7_tests.cpp:155-183."""
    h = np.array([[1.0, 0.0]], np.float32)
    w = np.array([[1, 3, 2], [0, 0, 0]], np.float32)
    rc, ids, sc = O.route(h, w, 2, 1, 1)
    assert rc == 0 and ids.tolist() == [[1, 2]] and abs(float(sc.sum()) - 1) < 1e-6
    rc, ids, _ = O.route(h, w, 1, 0, 0)
    assert ids.tolist() == [[1]]
    rc, ids, _ = O.route(h, np.array([[1, 1, 1], [0, 0, 0]], np.float32), 2, 1, 1)
    assert ids.tolist() == [[0, 1]], "ties by ascending expert id"
    rc, *_ = O.route(h, w, 4, 1, 1)
    assert rc == -1, "top-k greater than expert count is rejected"


def test_batch_router_grouping():
    """tests/phase8_tests.cpp:153-171 and phase12_tests.cpp:269-273."""
    h = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    w = np.array([[3, 2, 1], [0, 4, 1]], np.float32)
    rc, ids, sc = O.route(h, w, 2, 1, 1)
    assert ids[0].tolist() == [0, 1] and ids[1].tolist() == [1, 2]
    w12 = np.array([[3, 2, 0], [0, 2, 3]], np.float32)
    rc, ids, sc = O.route(h, w12, 2, 1, 1)
    counts, offsets, ptok, pw, slots = O.group(ids, sc, 3)
    assert [ptok[offsets[e]:offsets[e + 1]].tolist() for e in range(3)] == [[0, 2], [0, 1, 2], [1]]


def test_router_renorm_closed_form():
    """tests/phase18_19_tests.cpp:233-249: three experts, top-2, renorm; the
    selected scores equal softmax restricted to the pair."""
    h = np.array([[-2, -1], [0, 1], [2, 3]], np.float32)
    w = np.array([[2, 0, 1], [0, 2, 1]], np.float32)
    rc, ids, sc = O.route(h, w, 2, 1, 1)
    for t in range(3):
        logits = (h[t].astype(np.float64) @ w.astype(np.float64))
        e = np.exp(logits[ids[t]] - logits.max())
        np.testing.assert_allclose(sc[t], e / e.sum(), rtol=1e-6)


def test_topk_matches_brute_force():
    """Selection = the k smallest keys under (score desc, id asc), checked by
    enumerating every k-subset on small inputs with many ties."""
    rng = np.random.default_rng(1)
    for trial in range(60):
        E, k = int(rng.integers(2, 7)), 0
        k = int(rng.integers(1, E + 1))
        logits = rng.integers(-2, 3, E).astype(np.float32)  # heavy ties
        h = np.array([[1.0]], np.float32)
        w = logits.reshape(1, E)
        rc, ids, _ = O.route(h, w, k, 0, 0)
        best = None
        for combo in itertools.permutations(range(E), k):
            keyseq = [(-logits[e], e) for e in combo]
            if keyseq != sorted(keyseq):
                continue
            rest = [e for e in range(E) if e not in combo]
            if rest and max(((-logits[e], e) for e in combo)) > min(((-logits[e], e) for e in rest)):
                continue
            best = list(combo)
        assert ids[0].tolist() == best


def test_router_logits_sequential_double():
    """Logits = float of the double sum in ascending k: a different order
    (reversed) of the same double additions is not what the oracle computes
    whenever the two orders disagree."""
    rng = np.random.default_rng(2)
    h = rng.standard_normal((200, 512)).astype(np.float32)
    w = (0.02 * rng.standard_normal((512, 16))).astype(np.float32)
    rc, logits = O.router_logits(h, w)
    seq = np.zeros((200, 16))
    prod = h.astype(np.float64)[:, :, None] * w.astype(np.float64)[None]
    for kk in range(512):
        seq = seq + prod[:, kk, :]
    assert_bitexact(logits, seq.astype(np.float32), "sequential double logits")


def test_rmsnorm_closed_form():
    """tests/phase12_tests.cpp:182-198."""
    x = np.array([[3, 4], [0, 2]], np.float32)
    y = O.rmsnorm(x, np.array([1, 2], np.float32), 1e-6)
    a = np.float32(1 / math.sqrt(12.5 + 1e-6))
    b = np.float32(1 / math.sqrt(2.0 + 1e-6))
    np.testing.assert_allclose(y, [[3 * a, 8 * a], [0, 4 * b]], rtol=1e-6)


def test_combine_closed_form():
    """tests/phase18_19_tests.cpp:251-263: rows {2,0}, weights {0.5, 2}."""
    y = np.array([[2, 3], [-2, -1]], np.float32)  # grouped rows: expert 0 -> token 2, expert 1 -> token 0
    offsets = np.array([0, 1, 2], np.int32)
    ptok = np.array([2, 0], np.int32)
    pw = np.array([0.5, 2.0], np.float32)
    out = O.combine(y, offsets, ptok, pw, 3)
    assert out.tolist() == [[-4, -2], [0, 0], [1, 1.5]]


def test_combine_is_ascending_expert_float_sum():
    """MoERuntime.cpp:312-324: per token, float mul then add over groups in
    ascending expert id -- not rank order, not double."""
    rng = np.random.default_rng(4)
    T, k, E, W = 50, 4, 10, 33
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.uint32)
    sc = rng.random((T, k)).astype(np.float32)
    counts, offsets, ptok, pw, slots = O.group(ids, sc, E)
    yg = rng.standard_normal((T * k, W)).astype(np.float32)
    out = O.combine(yg, offsets, ptok, pw, T)
    ref = np.zeros((T, W), np.float32)
    for t in range(T):
        for e in sorted(ids[t].tolist()):
            r = int(np.where(ids[t] == e)[0][0])
            ref[t] = ref[t] + np.float32(sc[t, r]) * yg[slots[t, r]]
    assert_bitexact(out, ref, "combine")


def test_quantizer_properties():
    """tests/phase22_tests.cpp:164-203: determinism, zp = 0, error bound
    <= 0.5001 * scale; plus the textbook definition."""
    rng = np.random.default_rng(6)
    w = (0.02 * rng.standard_normal(10000)).astype(np.float32)
    q1, s1, z1, e1 = O.quantize_int8(w)
    q2, s2, z2, e2 = O.quantize_int8(w)
    assert np.array_equal(q1, q2) and s1 == s2 and z1 == z2 == 0
    assert e1 <= s1 * 0.5001
    assert np.float32(s1) == np.float32(np.abs(w).max()) / np.float32(127)
    expected = np.clip(np.sign(w / np.float32(s1)) * np.floor(np.abs(w / np.float32(s1)) + 0.5), -127, 127)
    assert np.array_equal(q1, expected.astype(np.int8)), "round half away from zero"
    qz, sz, zz, ez = O.quantize_int8(np.zeros(5, np.float32))
    assert sz == 1.0 and not qz.any()


def test_w8a32_phase23_inputs_vs_double():
    """tests/phase23_tests.cpp:189-240 inputs against an independent double
    accumulation of the same dequantised weights, 1e-5 + 1e-5|ref|."""
    for (r, kk, c) in [(1, 8, 8), (1, 257, 65), (2, 513, 33), (1, 1031, 31), (1, 2048, 768),
                       (1, 768, 2048), (3, 129, 7), (1, 4097, 67)]:
        i = np.arange(r * kk)
        x = (((i % 29) - 14).astype(np.float32) / np.float32(29.0)).reshape(r, kk)
        j = np.arange(kk * c)
        q = (((j * 13) % 255) - 127).astype(np.int8).reshape(kk, c)
        y = O.matmul_w8a32(x, q, 0.003, -3)
        wdq = (q.astype(np.float32) - np.float32(-3)) * np.float32(0.003)
        dbl = x.astype(np.float64) @ wdq.astype(np.float64)
        assert np.all(np.abs(y - dbl) <= 1e-5 + 1e-5 * np.abs(y))


def test_invalid_parameters_rejected():
    """validateParameters (Quantization.cpp:24-43)."""
    x = np.ones((1, 4), np.float32)
    q = np.ones((4, 2), np.int8)
    with pytest.raises(RuntimeError):
        O.matmul_w8a32(x, q, 0.0, 0)
    with pytest.raises(RuntimeError):
        O.matmul_w8a32(x, q, 1.0, 128)
    with pytest.raises(RuntimeError):
        O.rmsnorm(x, np.ones(4, np.float32), 0.0)
