"""The build-owned integer-limb INT8 arithmetic, on the CPU oracle.

Pins (no reference counterpart exists; the reference computes W8A32 in
FP32): digits reconstruct the fixed-point value exactly; the digit ranges and
the int32 bound hold; partials equal brute-force int64 dot products; the
limb result approaches the exact real-number product as L grows, and stays
within the north-star tolerance of the reference W8A32 path; the
recombination of the limb partials is pinned by hand-worked known answers
(ties to even, two roundings in top-limb-first order), by exactness where no
step rounds, and by its rounding-error bound."""
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


def _crafted_rows(plan):
    """Rows of integers whose three-limb digits and partials against one
    column are chosen by hand: each row holds 8355711 (= 127*65536 + 127*256
    + 127, the three-limb range, so the row's scale is exactly 1 and the
    quantiser keeps every integer as it is) against a zero weight, then
    entries (value, weight)."""
    K = 40
    x = np.zeros((len(plan), K), np.float32)
    q = np.zeros((K, 1), np.int8)
    x[:, 0] = 8355711.0
    for r, entries in enumerate(plan):
        for j, (value, weight) in enumerate(entries, start=1):
            x[r, j] = value
            assert q[j, 0] in (0, weight)
            q[j, 0] = weight
    return x, q


def test_limb_recombine_known_answers():
    """Known answers for the recombination of three limb partials (top limb
    first, each step rounded to float32, round-to-nearest-even), worked by
    hand on crafted partials, each chosen so that another order or a single
    rounding of the exact sum gives a different float:

      P = (100, 2, 131072): the top two limbs 256*2^17 + 2 = 2^25 + 2 lie
        halfway between the floats 2^25 and 2^25 + 4 (spacing 4), so they
        round to the even one, 2^25; then 2^33 + 100 rounds to 2^33 (spacing
        1024).  The exact sum 2^33 + 612 rounds to 2^33 + 1024, and so does
        low-limb-first (256*2 + 100 = 612 is exact).
      P = (-100, 6, 131072): 2^25 + 6 ties between 2^25 + 4 (odd) and
        2^25 + 8 (even): up, to 2^25 + 8; then 2^33 + 2048 - 100 = 2^33 + 1948
        rounds to 2^33 + 2048.  The exact sum 2^33 + 1436 rounds to 2^33 + 1024.
      the negation of the first row gives -2^33 (round-to-nearest is
        symmetric).
    The partials themselves come from the int64-pinned digit and partial
    routines; the result is multiplied by the row scale (1) and the weight
    scale (1 and 0.5, both exact)."""
    top = [(64 * 65536, 64)] * 32          # d2 = 64 against weight 64, 32 times: P2 = 2^17
    plan = [top + [(2 * 256, 1), (100, 1)],        # d1 = 2, then d0 = 100
            top + [(6 * 256, 1), (-100, 1)],
            [(-v, w) for v, w in top] + [(-2 * 256, 1), (-100, 1)]]
    x, q = _crafted_rows(plan)
    digits, s = O.limb_quantize(x, 3)
    assert np.array_equal(s, np.ones(3, np.float32))
    p = O.limb_partials(digits, q, 0)[:, :, 0]
    assert p[:, 0].tolist() == [100, 2, 131072]
    assert p[:, 1].tolist() == [-100, 6, 131072]
    assert p[:, 2].tolist() == [-100, -2, -131072]
    for scale in (np.float32(1.0), np.float32(0.5)):
        y = O.limb_matmul(x, q, scale, 0, 3)[:, 0]
        want = np.array([2.0 ** 33, 2.0 ** 33 + 2048, -2.0 ** 33], np.float64) * float(scale)
        assert y.astype(np.float64).tolist() == want.tolist(), (scale, y)


def test_limb_recombine_exact_when_representable():
    """Where every partial sum is an integer below 2^24 in magnitude no step
    rounds, so the result is exactly sum_l 256^l P_l times the scales: a
    dropped limb, a wrong limb weight or sign, swapped limb planes or a scale
    taken from the wrong row all change it.  The exact sum is formed in
    Python integers from int64 brute-force partials."""
    rng = np.random.default_rng(8)
    x = np.zeros((5, 96), np.float32)
    x[:, 0] = 8355711.0                 # scale exactly 1 (range of three limbs)
    x[:, 1:] = rng.integers(-2 ** 20, 2 ** 20, (5, 95)).astype(np.float32)
    q = rng.integers(-3, 4, (96, 6)).astype(np.int8)
    q[0] = 0
    q[rng.random((96, 6)) < 0.9] = 0    # few terms: the exact sums stay below 2^24
    digits, s = O.limb_quantize(x, 3)
    assert np.array_equal(s, np.ones(5, np.float32))
    p = np.einsum("lrk,kc->lrc", digits.astype(np.int64), q.astype(np.int64))
    exact = p[0] + 256 * p[1] + 65536 * p[2]
    small = (np.abs(exact) < 2 ** 24) & (np.abs(p[1] + 256 * p[2]) < 2 ** 24)
    assert small.mean() > 0.5 and (exact[small] != 0).any()
    rowscale = np.float32(2.0) ** np.arange(5, dtype=np.float32)[:, None]
    y = O.limb_matmul(x * rowscale, q, np.float32(0.25), 0, 3)   # scales 2^r * 0.25: exact
    want = exact * (2.0 ** np.arange(5)[:, None]) * 0.25
    assert np.array_equal(y.astype(np.float64)[small], want[small].astype(np.float64))


def test_limb_recombine_within_two_roundings():
    """On general data the result is within the error of its roundings: the
    top two limbs once (relative 2^-24, carried times 256 into the sum), the
    sum once, and the scale product once, of the exact integer sum."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 512)).astype(np.float32) * 50
    q = rng.integers(-128, 128, (512, 9)).astype(np.int8)
    digits, s = O.limb_quantize(x, 3)
    p = np.einsum("lrk,kc->lrc", digits.astype(np.int64), q.astype(np.int64))
    n1 = 256 * p[2] + p[1]
    exact = (256 * n1 + p[0]).astype(np.float64)
    alpha = (s.astype(np.float64) * 0.5)[:, None]
    y = O.limb_matmul(x, q, np.float32(0.5), 0, 3).astype(np.float64)
    u = 2.0 ** -24
    bound = alpha * (256 * u * np.abs(n1) + u * (np.abs(exact) + 256 * u * np.abs(n1))) \
        + u * np.abs(y) + 1e-300
    assert np.all(np.abs(y - exact * alpha) <= bound * 1.0001)
    # and the roundings are really there: the result is not the exact value
    assert (np.abs(y - exact * alpha) > 0).any()


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
