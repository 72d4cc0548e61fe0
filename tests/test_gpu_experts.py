"""GPU parity for the expert GEMMs (A5, A5', A6, A9) and the fused MoE block
(A11): bit-exact against the oracle's restatement of the limb arithmetic,
within tolerance against the reference W8A32 / FP32 numerics."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact, assert_compare, normwise, oracle_by_token_chunks
from hmoe import capi, synth
from hmoe.block import DeviceExpertLayer, MoEBlock

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,inner,cols,limbs,zp", [
    (1, 2048, 768, 2, 0), (5, 2048, 64, 3, 0), (16, 768, 2048, 2, -3), (3, 129, 7, 1, 5),
    (2, 4097, 67, 3, -128)])
def test_limb_partials_exact(dev, rows, inner, cols, limbs, zp):
    """INT8 int32 partials: device digits and partials equal the oracle's
    brute-force int64 dot products bit for bit."""
    rng = np.random.default_rng(inner + cols)
    x = (rng.standard_normal((rows, inner)) * 2).astype(np.float32)
    q = rng.integers(-128, 128, (inner, cols)).astype(np.int8)
    digits, scales = O.limb_quantize(x, limbs)
    ddig = dev.empty((limbs, rows, inner), np.int8)
    dsc = dev.empty(rows, np.float32)
    dev.call("hm_limb_quantize_rows", dev.to(x).data_ptr(), rows, inner, limbs, ddig.data_ptr(),
             dsc.data_ptr(), dev.stream)
    assert_bitexact(dev.host(ddig), digits, "digits")
    assert_bitexact(dev.host(dsc), scales, "row scales")
    part = dev.empty((limbs, rows, cols), np.int32)
    qt = np.ascontiguousarray(q.T)  # packed [cols x inner]
    dev.call("hm_limb_partials", ddig.data_ptr(), rows, inner, limbs, dev.to(qt).data_ptr(), zp,
             cols, part.data_ptr(), dev.stream)
    expected = O.limb_partials(digits, q, zp)
    brute = np.einsum("lrk,kc->lrc", digits.astype(np.int64), q.astype(np.int64) - zp)
    assert_bitexact(expected, brute.astype(np.int32), "oracle partials vs brute force")
    assert_bitexact(dev.host(part), expected, "device partials")


PHASE23_SHAPES = [(1, 8, 8), (1, 257, 65), (2, 513, 33), (1, 1031, 31), (1, 2048, 768),
                  (1, 768, 2048), (3, 129, 7), (1, 4097, 67)]


@pytest.mark.parametrize("rows,inner,cols", PHASE23_SHAPES)
def test_w8a32_reference_inputs(dev, rows, inner, cols):
    """tests/phase23_tests.cpp:189-240: x=((i%29)-14)/29, q=((i*13)%255)-127,
    {0.003, -3}.  Reference mode is bit-exact with the CPU path; cooperative
    (split-K) within 1e-5 + 1e-5|ref| and of an independent double oracle."""
    i = np.arange(rows * inner)
    x = (((i % 29) - 14).astype(np.float32) / np.float32(29.0)).reshape(rows, inner)
    j = np.arange(inner * cols)
    q = (((j * 13) % 255) - 127).astype(np.int8).reshape(inner, cols)
    cpu = O.matmul_w8a32(x, q, 0.003, -3)
    for mode in (1, 2, 0):
        plan = capi.HmInt8GemmPlan()
        capi.call("hm_plan_int8_gemm", rows, inner, cols, mode, C.byref(plan))
        scratch = dev.empty(max(1, plan.scratch_elements), np.float32)
        y = dev.empty((rows, cols), np.float32)
        dev.call("hm_matmul_w8a32", dev.to(x).data_ptr(), dev.to(q).data_ptr(), 0.003, -3,
                 y.data_ptr(), rows, inner, cols, mode, scratch.data_ptr(),
                 scratch.numel() * 4, dev.stream)
        got = dev.host(y)
        if plan.implementation == 1:
            assert_bitexact(got, cpu, f"reference mode {rows}x{inner}x{cols}")
        assert_compare(got, cpu, 1e-5, 1e-5, f"mode {mode} vs CPU")
        w = (q.astype(np.float32) - np.float32(-3)) * np.float32(0.003)
        dbl = x.astype(np.float64) @ w.astype(np.float64)
        assert np.all(np.abs(got - dbl) <= 1e-5 + 1e-5 * np.abs(cpu))


def test_matmul_f32_closed_form(dev):
    """tests/phase5_tests.cpp:147-160: [[1,2,3],[4,5,6]] x [[7,8],[9,10],[11,12]]."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    y = dev.empty((2, 2), np.float32)
    dev.call("hm_matmul_f32", dev.to(a).data_ptr(), dev.to(b).data_ptr(), y.data_ptr(), 2, 3, 2,
             dev.stream)
    assert dev.host(y).tolist() == [[58, 64], [139, 154]]


def test_elementwise(dev):
    """SiLU bit-exact with Activation.cpp:44 (glibc expf); mul/add exact."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(100003) * 8).astype(np.float32)
    b = rng.standard_normal(100003).astype(np.float32)
    y = dev.empty(x.shape, np.float32)
    dev.call("hm_silu", dev.to(x).data_ptr(), y.data_ptr(), x.size, dev.stream)
    assert_bitexact(dev.host(y), O.silu(x), "silu")
    dev.call("hm_mul", dev.to(x).data_ptr(), dev.to(b).data_ptr(), y.data_ptr(), x.size, dev.stream)
    assert_bitexact(dev.host(y), x * b, "mul")
    dev.call("hm_add", dev.to(x).data_ptr(), dev.to(b).data_ptr(), y.data_ptr(), x.size, dev.stream)
    assert_bitexact(dev.host(y), x + b, "add")


def _tiles(w_kn: np.ndarray) -> np.ndarray:
    """The kernels' INT8 tile layout of one projection W [K x N] (K inner):
    zero-padded to multiples of 32, tile (n // 32, k // 32) at
    ((n // 32) * K32/32 + k // 32) KB, inside it lane n % 32 + 32 ((k // 16) % 2)
    holding the 16 bytes k % 16 = 0..15."""
    K, N = w_kn.shape
    K32, N32 = -(-K // 32) * 32, -(-N // 32) * 32
    p = np.zeros((K32, N32), np.int8)
    p[:K, :N] = w_kn
    t = p.reshape(K32 // 32, 2, 16, N32 // 32, 32)     # kb, half, j, cb, col
    return np.ascontiguousarray(t.transpose(3, 0, 1, 4, 2)).reshape(-1)  # cb, kb, half, col, j


@pytest.mark.parametrize("E,H,I", [(3, 40, 70), (2, 2048, 768)])
def test_pack_layer_tile_layout(dev, E, H, I):
    """hm_pack_layer writes every INT8 projection as 32 x 32 tiles in the MFMA
    B-operand order (one wave-wide 16-byte load = one contiguous kilobyte),
    projections gate | up | down of each expert back to back, padding zero."""
    rng = np.random.default_rng(E * H)
    payload = rng.integers(-128, 128, (E, 3, H * I)).astype(np.int8)
    nbytes = capi.load().hm_packed_layer_bytes(E, H, I, capi.HM_DTYPE_INT8)
    packed = dev.empty(nbytes, np.uint8)
    dev.call("hm_pack_layer", dev.to(payload).data_ptr(), E, H, I, capi.HM_DTYPE_INT8,
             packed.data_ptr(), dev.stream)
    got = dev.host(packed).view(np.int8)
    expected = np.concatenate([
        _tiles(payload[e, p].reshape(H, I) if p < 2 else payload[e, p].reshape(I, H))
        for e in range(E) for p in range(3)])
    assert_bitexact(got, expected, "tile layout")


def _layer_inputs(seed, T, H, E, I, int8, skew=False):
    payload, scale, zp = synth.expert_layer(seed, 0, E, H, I, int8)
    h = O.rmsnorm(synth.raw_hidden(seed, T, H), np.ones(H, np.float32))
    w = synth.router_weights(seed, 0, H, E)
    if skew:
        synth.apply_skew(h, w, synth.zipf_bias(seed, E))
    return payload, scale, zp, h, w


BLOCK_CASES = [  # (T, H, E, I, k, X digits, Z digits) -- MFMA shapes and generic shapes
    (1, 2048, 128, 768, 8, 2, 3), (4, 2048, 128, 768, 8, 3, 3), (16, 2048, 128, 768, 8, 2, 2),
    (70, 512, 16, 256, 4, 2, 3), (5, 64, 8, 32, 2, 2, 2), (6, 96, 5, 40, 3, 3, 3), (3, 2, 3, 2, 2, 2, 3),
    # several row tiles per expert (ragged last tile) through the MFMA kernels
    (300, 2048, 4, 768, 2, 2, 3), (300, 2048, 4, 768, 2, 3, 2), (203, 1024, 3, 384, 2, 3, 3),
    (90, 1024, 6, 512, 3, 2, 3), (150, 512, 2, 128, 1, 1, 1), (300, 512, 4, 256, 2, 2, 3),
    # more than 1024 pairs with E % 64 == 0: the prefill router's select
    # kernel counts the permutation's chunk histograms (the count pass is
    # skipped)
    (160, 2048, 64, 768, 8, 2, 3), (160, 512, 64, 256, 8, 2, 2)]


@pytest.mark.parametrize("T,H,E,I,k,LX,LZ", BLOCK_CASES)
def test_block_int8_bitexact_vs_limb_oracle(dev, T, H, E, I, k, LX, LZ):
    print(f"[gpu] block int8 T={T} H={H} E={E} I={I} k={k} limbs=({LX}, {LZ})", flush=True)
    payload, scale, zp, h, w = _layer_inputs(11 + T, T, H, E, I, True)
    layer = DeviceExpertLayer(payload, scale, zp, H, I)
    block = MoEBlock(layer, k, limbs_x=LX, limbs_z=LZ)
    # the limb arithmetic at every batch size (decode sizes default to the GEMV)
    res = block.execute_batch(dev.to(h), dev.to(w), exec_flags=capi.HM_EXEC_LIMBS)
    out = dev.host(res.output)
    lout, lids, lsc = O.moe_block_limbs(payload, scale, zp, h, w, k, I, LX, LZ)
    assert_bitexact(res.ids, lids, "ids")
    assert_bitexact(res.scores, lsc, "scores")
    assert_bitexact(out, lout, "block output vs limb oracle")
    # generic (scalar) kernels give the same bits
    res2 = block.execute_batch(dev.to(h), dev.to(w), exec_flags=capi.HM_EXEC_GENERIC)
    assert_bitexact(dev.host(res2.output), out, "MFMA vs generic kernels")
    if T <= capi.HM_GEMV_MAX_TOKENS:
        # the default decode path: the W8A32 GEMV in FP32 up to
        # HM_GEMV_MAX_PAIRS pairs (against the reference), the limb GEMMs
        # beyond (the same bits as above)
        rout_, _, _ = O.moe_block(payload, scale, zp, h, w, k, I)
        gres = block.execute_batch(dev.to(h), dev.to(w))
        assert_bitexact(gres.ids, res.ids, "default decode path routing")
        if T * k <= capi.HM_GEMV_MAX_PAIRS:
            assert_compare(dev.host(gres.output), rout_, 1e-4, 1e-4,
                           "GEMV block vs reference (1e-4)")
        else:
            assert_bitexact(dev.host(gres.output), out, "default decode path vs limb GEMMs")
    # reference W8A32 numerics
    rout, rids, rsc = O.moe_block(payload, scale, zp, h, w, k, I)
    assert_bitexact(res.ids, rids, "ids vs reference path")
    counts, offsets, ptok, pw, _ = O.group(rids, rsc, E)
    assert_bitexact(res.perm_tokens, ptok, "permutation vs reference path")
    nw = normwise(out, rout)
    if min(LX, LZ) == 1:  # one digit = plain int8 activations: W8A8 accuracy
        assert nw < 5e-2
    elif LX >= 2 and LZ >= 3:
        # the block's default digit counts
        assert_compare(out, rout, 1e-4, 1e-4, "block vs reference W8A32 (1e-4)")
        assert nw < 1e-4
        if LX == 3:
            assert_compare(out, rout, 1e-5, 1e-5, "three-digit block vs reference W8A32 (1e-5)")
    else:  # two Z digits with one scale per row: about 16-bit Z
        assert nw < 3e-4


@pytest.mark.parametrize("T,H,E,I,k,LX,LZ,skew", [
    (400, 1024, 16, 512, 4, 2, 3, True), (256, 2048, 128, 768, 8, 3, 3, False),
    (256, 512, 32, 256, 8, 1, 2, True)])
def test_block_skinny_split_k(dev, T, H, E, I, k, LX, LZ, skew):
    """With HM_EXEC_SPLIT_K, experts of at most 32 grouped rows run the
    bounded split-K kernel (K split over the workgroup's waves, int32 limb
    partials summed exactly), the others the tile kernels, in one block: a
    skewed batch with both kinds, a mid-size batch where most experts are
    skinny, one to three digit planes.  Bit-exact against the limb oracle,
    against the generic kernels and against the tile kernels alone."""
    print(f"[gpu] skinny split-K T={T} H={H} E={E} I={I} k={k} limbs=({LX}, {LZ})", flush=True)
    payload, scale, zp, h, w = _layer_inputs(41 + T, T, H, E, I, True, skew=skew)
    block = MoEBlock(DeviceExpertLayer(payload, scale, zp, H, I), k, limbs_x=LX, limbs_z=LZ)
    res = block.execute_batch(dev.to(h), dev.to(w),
                              exec_flags=capi.HM_EXEC_LIMBS | capi.HM_EXEC_SPLIT_K)
    counts = np.asarray(res.counts)
    assert ((counts > 0) & (counts <= 32)).any(), "no skinny group in this batch"
    if skew:
        assert (counts > 32).any(), "no tiled group in this batch"
    out = dev.host(res.output)
    lout, lids, _ = O.moe_block_limbs(payload, scale, zp, h, w, k, I, LX, LZ)
    assert_bitexact(res.ids, lids, "ids")
    assert_bitexact(out, lout, "split-K block vs limb oracle")
    gen = block.execute_batch(dev.to(h), dev.to(w), exec_flags=capi.HM_EXEC_GENERIC)
    assert_bitexact(dev.host(gen.output), out, "split-K kernels vs generic kernels")
    tiles = block.execute_batch(dev.to(h), dev.to(w), exec_flags=capi.HM_EXEC_LIMBS)
    assert_bitexact(dev.host(tiles.output), out, "split-K kernels vs tile kernels")


def test_block_int8_nonzero_zero_points(dev):
    """Zero points other than 0 (validateParameters allows [-128, 127])."""
    T, H, E, I, k = 24, 2048, 8, 768, 2
    payload, scale, zp, h, w = _layer_inputs(5, T, H, E, I, True)
    zp = np.random.default_rng(1).integers(-5, 6, zp.shape).astype(np.int32)
    layer = DeviceExpertLayer(payload, scale, zp, H, I)
    block = MoEBlock(layer, k, limbs_x=2, limbs_z=3)
    out = dev.host(block.execute_batch(dev.to(h), dev.to(w)).output)
    lout, _, _ = O.moe_block_limbs(payload, scale, zp, h, w, k, I, 2, 3)
    assert_bitexact(out, lout, "block with zero points vs limb oracle")
    # decode-size batch with zero points through the GEMV
    hs = np.ascontiguousarray(h[:5])
    gout = dev.host(block.execute_batch(dev.to(hs), dev.to(w)).output)
    rout, _, _ = O.moe_block(payload, scale, zp, hs, w, k, I)
    assert_compare(gout, rout, 1e-4, 1e-4, "GEMV with zero points vs reference (1e-4)")
    gen = block.execute_batch(dev.to(h), dev.to(w), exec_flags=capi.HM_EXEC_GENERIC)
    assert_bitexact(dev.host(gen.output), out, "MFMA vs generic with zero points")


@pytest.mark.parametrize("T,H,E,I,k,skew", [
    (1, 2048, 128, 768, 8, False), (4, 2048, 128, 768, 8, False), (8, 2048, 128, 768, 8, True),
    (16, 512, 4, 256, 2, False), (13, 1024, 3, 512, 3, False), (9, 256, 2, 1024, 1, False),
    (16, 256, 64, 1024, 4, False), (5, 528, 6, 400, 2, False), (2, 2048, 128, 768, 8, False),
    (3, 256, 8, 96, 5, False), (1, 1024, 16, 512, 1, False), (1, 128, 4, 32, 1, False),
    (3, 1024, 16, 512, 8, False)])
def test_block_gemv_decode(dev, T, H, E, I, k, skew):
    """Decode-size blocks of at most HM_GEMV_MAX_PAIRS pairs take the W8A32
    GEMV (FP32): ids bit-exact, output
    within 1e-4 of the reference; several rows per expert (the register
    row blocks), skewed groups, every supported K length, the four-column-
    tile down workgroups (32 or more active experts) at their largest K, and
    H, I off the 32-column tile grid (zero-padded K tiles, a partial last
    column tile).  With T*k <= 16 the down projection and the combine run as
    one kernel: one active expert (sixteen waves on its K range; with I=32
    fifteen of them have no K tile), eight, and sixteen (one wave per
    expert, K in two register chunks).  Three tokens at top-8 over sixteen
    experts (24 pairs) take the separate down GEMV and combine with twelve
    to sixteen active experts."""
    print(f"[gpu] gemv T={T} H={H} E={E} I={I} k={k} skew={skew}", flush=True)
    payload, scale, zp, h, w = _layer_inputs(7 + T, T, H, E, I, True, skew=skew)
    block = MoEBlock(DeviceExpertLayer(payload, scale, zp, H, I), k)
    res = block.execute_batch(dev.to(h), dev.to(w))
    rout, rids, rsc = O.moe_block(payload, scale, zp, h, w, k, I)
    assert_bitexact(res.ids, rids, "ids")
    assert_bitexact(res.scores, rsc, "scores")
    out = dev.host(res.output)
    assert_compare(out, rout, 1e-4, 1e-4, "GEMV block vs reference W8A32 (1e-4)")
    assert normwise(out, rout) < 1e-5
    # per-expert outputs: the grouped rows equal the reference expert MLP
    y = dev.host(res.expert_out)
    for b in res.batches[:4]:
        lo = int(res.offsets[b.expert_id])
        xe = np.ascontiguousarray(h[b.token_indices])
        ref = O.expert_mlp(payload, scale, zp, b.expert_id, xe, I)
        assert_compare(y[lo:lo + len(b.token_indices)], ref, 1e-4, 1e-4, "expert rows")


@pytest.mark.parametrize("T,skew", [(16, True), (9, False)])
def test_block_limb_decode(dev, T, skew):
    """Decode-size blocks of more than HM_GEMV_MAX_PAIRS pairs (C3-16: 128
    pairs over about 80 experts) take the limb GEMMs, their activation digits
    cut by the fused decode router's select kernel: output bit-exact against
    the limb oracle and within 1e-4 of the reference, routing and grouping
    bit-exact."""
    H, E, I, k = 2048, 128, 768, 8
    assert T * k > capi.HM_GEMV_MAX_PAIRS
    print(f"[gpu] limb decode T={T} skew={skew}", flush=True)
    payload, scale, zp, h, w = _layer_inputs(29 + T, T, H, E, I, True, skew=skew)
    block = MoEBlock(DeviceExpertLayer(payload, scale, zp, H, I), k)
    res = block.execute_batch(dev.to(h), dev.to(w))
    lout, lids, lsc = O.moe_block_limbs(payload, scale, zp, h, w, k, I, block.limbs_x,
                                        block.limbs_z)
    assert_bitexact(res.ids, lids, "ids")
    assert_bitexact(res.scores, lsc, "scores")
    out = dev.host(res.output)
    assert_bitexact(out, lout, "block output vs limb oracle")
    _, _, ptok, _, _ = O.group(lids, lsc, E)
    assert_bitexact(res.perm_tokens, ptok, "grouping")
    rout, _, _ = O.moe_block(payload, scale, zp, h, w, k, I)
    assert_compare(out, rout, 1e-4, 1e-4, "limb decode block vs reference W8A32 (1e-4)")


@pytest.mark.parametrize("T,E", [(16, 64), (1, 64), (5, 8), (40, 8), (300, 4)])
def test_block_fp32_vs_reference(dev, T, E):
    """FP32 experts (C1 shape): within 1e-3 of the reference (north star).
    T <= 16 takes the FP32 GEMV (T = 5, E = 8: five rows on most experts,
    two LDS passes); T=300 with E=4, k=2 puts about 150 rows on each
    expert: several 64-row matrix-core tiles per expert with a ragged last
    tile."""
    H, I, k = 2048, 768, 8 if E >= 8 else 2
    print(f"[gpu] fp32 block T={T} E={E} k={k}", flush=True)
    payload, scale, zp, h, w = _layer_inputs(3, T, H, E, I, False)
    layer = DeviceExpertLayer(payload, None, None, H, I)
    block = MoEBlock(layer, k)
    res = block.execute_batch(dev.to(h), dev.to(w))
    rout, rids, rsc = oracle_by_token_chunks(O.moe_block, h, payload, scale, zp, w, k, I)
    assert_bitexact(res.ids, rids, "ids")
    assert_bitexact(res.scores, rsc, "scores")
    if T > 64:
        assert int(np.bincount(rids.ravel(), minlength=E).max()) > 64
    assert_compare(dev.host(res.output), rout, 1e-3, 1e-3, "fp32 block (1e-3)")
    assert normwise(dev.host(res.output), rout) < 1e-5


def test_block_c4_prefill_properties(dev):
    """C4 at full size (T=4096, skewed): routing bit-exact against the
    oracle, MFMA == generic on a token subset is covered above; here:
    determinism across runs, finite output, and exact linearity of the
    combine over a duplicated batch."""
    cfg = synth.CONFIGS["C4"]
    T, H, E, I, k = cfg.tokens, cfg.hidden, cfg.experts, cfg.inter, cfg.top_k
    payload, scale, zp, h, w = _layer_inputs(cfg.seed, T, H, E, I, True, skew=True)
    layer = DeviceExpertLayer(payload, scale, zp, H, I)
    block = MoEBlock(layer, k, limbs_x=2, limbs_z=3)
    r1 = block.execute_batch(dev.to(h), dev.to(w))
    o1 = dev.host(r1.output).copy()
    r2 = block.execute_batch(dev.to(h), dev.to(w))
    assert_bitexact(dev.host(r2.output), o1, "run-to-run determinism")
    assert np.isfinite(o1).all()
    rc, ids, scores = O.route(h, w, k, 1, 1)
    assert_bitexact(r1.ids, ids, "C4 ids")
    assert_bitexact(r1.scores, scores, "C4 scores")
    # the permutation (its chunk histograms counted by the prefill select
    # kernel at this size) against the oracle's grouping, bit for bit
    counts, offsets, ptok, pw, _ = O.group(ids, scores, E)
    assert_bitexact(r1.offsets, offsets, "C4 offsets")
    assert_bitexact(r1.perm_tokens, ptok, "C4 permutation")
    assert_bitexact(r1.perm_weights, pw, "C4 permuted weights")
    # a token's output depends only on its own row: a 64-token slice run alone
    # gives the same bits (routing, permutation and tiling are per token/row)
    sub = slice(1000, 1064)
    r3 = block.execute_batch(dev.to(np.ascontiguousarray(h[sub])), dev.to(w))
    assert_bitexact(dev.host(r3.output), o1[sub], "token-slice invariance")
    lout, _, _ = O.moe_block_limbs(payload, scale, zp, np.ascontiguousarray(h[sub]), w, k, I, 2, 3)
    assert_bitexact(o1[sub], lout, "C4 slice vs limb oracle")
    # every token against the reference W8A32 block
    rout, _, _ = oracle_by_token_chunks(O.moe_block, h, payload, scale, zp, w, k, I)
    assert_compare(o1, rout, 1e-4, 1e-4, "C4 full batch vs reference W8A32 (1e-4)")
    nw = normwise(o1, rout)
    print(f"[gpu] C4 full batch normwise error {nw:.3e}", flush=True)
    assert nw < 1e-4


def test_block_one_token_select_at_rounding_boundaries(dev):
    """One token on the GEMV path: every workgroup of the gate/up launch
    redoes the select (select_gateup_kernel).  Logits the bound cannot
    settle (experts 0-3: 1 + 2^-24, an exact tie that rounds to 1.0) take
    the reference's chain inside that kernel; ids and scores bit-exact
    against the reference, the output within 1e-4, and the sequential-chain
    flag gives the same bits."""
    from hmoe import capi
    H, E, I, k = 256, 64, 64, 2
    rng = np.random.default_rng(5)
    payload, scale, zp = synth.expert_layer(21, 0, E, H, I, True)
    h = np.zeros((1, H), np.float32)
    w = np.zeros((H, E), np.float32)
    h[0, 0], h[0, 1] = 1.0, 2.0 ** -24
    h[0, 2:] = rng.standard_normal(H - 2).astype(np.float32)
    w[0, :], w[1, :] = 1.0, 1.0
    w[2:, 4:] = (0.02 * rng.standard_normal((H - 2, E - 4))).astype(np.float32)
    block = MoEBlock(DeviceExpertLayer(payload, scale, zp, H, I), k)
    res = block.execute_batch(dev.to(h), dev.to(w))
    rout, rids, rsc = O.moe_block(payload, scale, zp, h, w, k, I)
    assert_bitexact(res.ids, rids, "ids")
    assert_bitexact(res.scores, rsc, "scores")
    out = dev.host(res.output)
    assert_compare(out, rout, 1e-4, 1e-4, "one-token block vs reference (1e-4)")
    seq = block.execute_batch(dev.to(h), dev.to(w), exec_flags=capi.HM_EXEC_ROUTE_SEQUENTIAL)
    assert_bitexact(seq.ids, res.ids, "ids, sequential chains")
    assert_bitexact(dev.host(seq.output), out, "output, sequential chains")


def test_block_one_token_nonfinite_score(dev):
    """A non-finite router score at one token (the select inside the gate/up
    launch) sets HM_STATUS_NONFINITE_SCORE, as CpuRouterBackend.cpp:47
    throws; the block raises, and the next call on clean weights is right."""
    H, E, I, k = 256, 64, 64, 2
    payload, scale, zp, h, w = _layer_inputs(23, 1, H, E, I, True)
    block = MoEBlock(DeviceExpertLayer(payload, scale, zp, H, I), k)
    bad = w.copy()
    bad[3, 5] = np.inf
    from hmoe import capi
    with pytest.raises(RuntimeError, match="status bits") as err:
        block.execute_batch(dev.to(h), dev.to(bad))
    bits = int(str(err.value).split("status bits ")[1].rstrip(")"), 16)
    assert bits & capi.HM_STATUS_NONFINITE_SCORE
    res = block.execute_batch(dev.to(h), dev.to(w))
    rout, rids, _ = O.moe_block(payload, scale, zp, h, w, k, I)
    assert_bitexact(res.ids, rids, "ids after the failed call")
    assert_compare(dev.host(res.output), rout, 1e-4, 1e-4, "output after the failed call")


@pytest.mark.parametrize("T", [1, 16, 300])
def test_block_graph_replay(dev, T):
    """The block's launch sequence captured as one HIP graph (kernels only:
    no memset or copy nodes) replays to the eager result every time, with
    eager work and synchronisations between the replays."""
    import torch
    print(f"[gpu] graph replay T={T}", flush=True)
    H, E, I, k = 2048, 128, 768, 8
    payload, scale, zp, h, w = _layer_inputs(31 + T, T, H, E, I, True)
    block = MoEBlock(DeviceExpertLayer(payload, scale, zp, H, I), k)
    dh, dw = dev.to(h), dev.to(w)
    eager = block.launch(dh, dw)["out"].clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        block.launch(dh, dw)
    for i in range(3):
        block._io_bufs["out"].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(block._io_bufs["out"], eager), f"replay {i} differs"
        # eager work between replays
        again = block.launch(dh, dw)["out"]
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
