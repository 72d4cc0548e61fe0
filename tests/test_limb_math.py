"""The build-owned integer-limb INT8 arithmetic, on the CPU oracle.

Pins (no reference counterpart exists; the reference computes W8A32 in
FP32): digits reconstruct the fixed-point value exactly; the digit ranges and
the int32 bound hold; partials equal brute-force int64 dot products; the
limb result approaches the exact real-number product as L grows, and stays
within the north-star tolerance of the reference W8A32 path."""
from __future__ import annotations

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact, assert_compare, normwise

RANGE = {1: 127, 2: 32639, 3: 8355711}


@pytest.mark.parametrize("limbs", [1, 2, 3])
def test_digits_reconstruct_fixed_point(limbs):
    rng = np.random.default_rng(limbs)
    x = (rng.standard_normal((20, 777)) * rng.uniform(1e-3, 1e3, (20, 1))).astype(np.float32)
    x[3] = 0.0
    x[4, ::7] = 0.0
    digits, scales = O.limb_quantize(x, limbs)
    assert digits.min() >= -128 and digits.max() <= 127
    n = sum(digits[l].astype(np.int64) * 256 ** l for l in range(limbs))
    assert np.abs(n).max() <= RANGE[limbs]
    amax = np.abs(x).max(axis=1)
    inv = np.where(amax > 0, np.float32(RANGE[limbs]) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    expected_n = np.clip(np.rint((x * inv[:, None]).astype(np.float32)), -RANGE[limbs], RANGE[limbs])
    assert np.array_equal(n, expected_n.astype(np.int64)), "n = clamp(rint(x * inv))"
    assert scales[3] == 0.0 and not digits[:, 3].any()
    # |x - n*s| <= s/2 + |x| * 3 * 2^-24: the fixed-point representation error
    # plus the float roundings of inv, x*inv and s
    recon = n * scales[:, None].astype(np.float64)
    err = np.abs(x - recon)
    assert np.all(err <= 0.5 * scales[:, None] + np.abs(x) * 3 * 2.0 ** -24 + 1e-30)


@pytest.mark.parametrize("limbs,zp", [(1, 0), (2, -3), (3, 7), (2, -128)])
def test_partials_equal_int64_brute_force(limbs, zp):
    rng = np.random.default_rng(10 + limbs)
    x = rng.standard_normal((6, 300)).astype(np.float32)
    q = rng.integers(-128, 128, (300, 11)).astype(np.int8)
    digits, _ = O.limb_quantize(x, limbs)
    p = O.limb_partials(digits, q, zp)
    brute = np.einsum("lrk,kc->lrc", digits.astype(np.int64), q.astype(np.int64) - zp)
    assert_bitexact(p, brute.astype(np.int32), "partials")


def test_partial_bound_fits_int32():
    """|P| <= K * 128 * 255 < 2^31 for K <= 65793 (worst-case digits)."""
    K = 2048
    digits = np.full((1, 1, K), -128, np.int8)
    q = np.full((K, 1), 127, np.int8)
    p = O.limb_partials(digits, q, -128)
    assert int(p[0, 0, 0]) == -128 * 255 * K
    assert 65793 * 128 * 255 < 2 ** 31


@pytest.mark.parametrize("limbs", [1, 2, 3])
def test_limb_matmul_converges(limbs):
    """Error against the exact product of the dequantised weights shrinks
    about 256x per limb."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 2048)).astype(np.float32)
    # packer-quantised N(0, 0.02) weights, as in the configs
    q, scale, _, _ = O.quantize_int8((0.02 * rng.standard_normal((2048, 64))).astype(np.float32))
    scale = np.float32(scale)
    y = O.limb_matmul(x, q, scale, 0, limbs)
    exact = x.astype(np.float64) @ (q.astype(np.float64) * float(scale))
    e = normwise(y, exact)
    assert e < {1: 3e-2, 2: 2e-4, 3: 2e-6}[limbs], e
    w8 = O.matmul_w8a32(x, q, scale, 0)
    if limbs >= 2:
        assert_compare(y, w8, 1e-4, 1e-4, f"L={limbs} vs W8A32")


def test_limb_block_within_north_star_tolerance():
    """The limb MoE block at a reduced Qwen shape: L=2 within 1e-4 and L=3
    within 1e-5 (compare form) of the reference W8A32 block."""
    from hmoe import synth
    E, H, I, T, k = 16, 2048, 768, 6, 4
    payload, scale, zp = synth.expert_layer(9, 0, E, H, I, True)
    h = O.rmsnorm(synth.raw_hidden(9, T, H), np.ones(H, np.float32))
    w = synth.router_weights(9, 0, H, E)
    ref, rids, _ = O.moe_block(payload, scale, zp, h, w, k, I)
    for L, tol in ((2, 1e-4), (3, 1e-5)):
        out, ids, _ = O.moe_block_limbs(payload, scale, zp, h, w, k, I, L, L)
        assert_bitexact(ids, rids, "routing is independent of the limb count")
        assert_compare(out, ref, tol, tol, f"L={L}")


def test_limb_recombine_is_the_documented_sequence():
    """recombine: c = float(P2); c = fmaf(c, 256, float(P1)); ...  A recombination
    in a different order (low limb first) is not bit-identical in general;
    the oracle uses the documented order."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((4, 512)).astype(np.float32) * 50
    q = rng.integers(-127, 128, (512, 9)).astype(np.int8)
    digits, s = O.limb_quantize(x, 3)
    p = O.limb_partials(digits, q, 0).astype(np.float32)
    c = p[2]
    for l in (1, 0):
        c = (c.astype(np.float64) * 256 + p[l].astype(np.float64)).astype(np.float32)  # fma: one rounding
    y = c * (s[:, None] * np.float32(0.5))
    assert_bitexact(O.limb_matmul(x, q, np.float32(0.5), 0, 3), y.astype(np.float32), "recombine")


def test_c4_full_batch_error_budget():
    """The block's default limb counts (two X digits, three Z digits) at the
    full C4 workload (T=4096, E=128, k=8, Zipf-skewed routing) against the
    reference W8A32 block on every token: the compare form at 1e-4
    (CorrectnessOracle.cpp:44-67) and the normwise error max|a-b| / max|b|
    below 1e-4 with at least 20 % to spare.  The device path is bit-exact
    against this limb arithmetic, so this bounds the device's error at the
    benchmark workload, not only on a sample."""
    from conftest import oracle_by_token_chunks
    from hmoe import synth
    cfg = synth.CONFIGS["C4"]
    T, H, E, I, k = cfg.tokens, cfg.hidden, cfg.experts, cfg.inter, cfg.top_k
    payload, scale, zp = synth.expert_layer(cfg.seed, 0, E, H, I, True)
    h = O.rmsnorm(synth.raw_hidden(cfg.seed, T, H), np.ones(H, np.float32))
    w = synth.router_weights(cfg.seed, 0, H, E)
    synth.apply_skew(h, w, synth.zipf_bias(cfg.seed, E))
    ref, rids, _ = oracle_by_token_chunks(O.moe_block, h, payload, scale, zp, w, k, I)
    out, ids, _ = oracle_by_token_chunks(O.moe_block_limbs, h, payload, scale, zp, w, k, I, 2, 3)
    assert_bitexact(ids, rids, "routing")
    err = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    tok = int(np.argmax(err.max(axis=1)))
    nw = normwise(out, ref)
    per_token = err.max(axis=1) / np.maximum(np.abs(ref).max(axis=1), 1e-30)
    print(f"C4 limbs (2, 3): normwise {nw:.3e}, worst token {tok} (abs {err.max():.3e}, "
          f"its own normwise {per_token[tok]:.3e}), worst per-token normwise "
          f"{per_token.max():.3e} at token {int(np.argmax(per_token))}")
    assert_compare(out, ref, 1e-4, 1e-4, "C4 limbs (2, 3) vs reference W8A32")
    assert nw < 0.8e-4, nw
