"""hm_moe_layer_forward: the MoE sub-layer of the transformer block,
out = h + MoE(RMSNorm(h)) (src/transformer/runtime/TransformerBlock.cpp:
88-104), with the RMSNorm (src/transformer/norm/RMSNorm.cpp:65-77) folded
into the decode router's first kernel.  Called through the C ABI and
checked bit for bit: its normalised rows against the oracle's RMSNorm, its
routing and output against hm_rmsnorm followed by hm_moe_block_forward with
h as the residual.  Decode sizes take the folded norm, prefill sizes the
separate launch; gamma is not all ones; HM_EXEC_ROUTE_SEQUENTIAL makes every
row take the sequential sum of squares; and row 0 is built so that some
elements are not settled by the bracket around the tree sum, which sends
their K blocks to the sequential sum."""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact
from hmoe import capi, synth
from hmoe.block import DeviceExpertLayer, MoEBlock

pytestmark = pytest.mark.gpu

H, E, I, K = 2048, 32, 256, 4
EPS = 1e-5


def _slack(width):
    """The kernels' relative bracket half-width around the tree sum of
    `width` squares (the same double operations in the same order)."""
    u = 2.0 ** -53
    gam = (width - 1) * u / (1.0 - (width - 1) * u)
    return 4.0 * gam / (1.0 - gam)


def _unsettled_row(rng, eps):
    """A row whose squares add exactly in any order (powers of two), and a
    gamma with 32 elements (one per router K block) where float(x * inv * g)
    differs at the two ends of the bracket, so the kernels must take the
    sequential sum there.  Returns (row, gamma, unsettled indices)."""
    row = (rng.choice([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], H)).astype(np.float32)
    gamma = (0.5 + rng.random(H)).astype(np.float32)
    s = float(np.sum(row.astype(np.float64) ** 2))  # exact
    d = _slack(H)
    inv_lo = 1.0 / math.sqrt(s * (1.0 + d) / H + float(np.float32(eps)))
    inv_hi = 1.0 / math.sqrt(s * (1.0 - d) / H + float(np.float32(eps)))
    # candidate gammas: every float in [1, 2).  Every x here is a power of
    # two, so x * inv * g scales inv * g exactly and rounds like it.
    g = 1.0 + np.arange(1 << 23, dtype=np.float64) * 2.0 ** -23
    hits = np.nonzero((inv_lo * g).astype(np.float32) != (inv_hi * g).astype(np.float32))[0]
    assert hits.size >= 32, "too few unsettled gammas for this row"
    picked = []
    for blk in range(32):
        i = blk * (H // 32) + int(rng.integers(H // 32))
        gamma[i] = np.float32(g[hits[int(rng.integers(hits.size))]])
        picked.append(i)
    return row, gamma, picked


@pytest.fixture(scope="module")
def layer():
    payload, scale, zp = synth.expert_layer(91, 0, E, H, I, True)
    return DeviceExpertLayer(payload, scale, zp, H, I)


def _layer_forward(block, h, gamma, w, flags, normed_offset=0):
    """normed_offset: the normalised rows start that many floats into their
    buffer (an offset of 1 leaves them 4-byte but not 16-byte aligned)."""
    import torch
    T, width = h.shape
    P = T * block.top_k
    normed_buf = torch.full((T * width + normed_offset,), float("nan"), dtype=torch.float32,
                            device="cuda")
    normed = normed_buf[normed_offset:].view(T, width)
    out = torch.full((T, width), float("nan"), dtype=torch.float32, device="cuda")
    ids = torch.full((T, block.top_k), -1, dtype=torch.int32, device="cuda")
    scores = torch.empty((T, block.top_k), dtype=torch.float32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    need = capi.load().hm_moe_block_workspace_bytes(C.byref(block.layer.desc), T, block.top_k,
                                                    block.limbs_x, block.limbs_z,
                                                    block.flags | flags)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    io = capi.HmBlockIO(out.data_ptr(), ids.data_ptr(), scores.data_ptr(), None, None, None,
                        None, None, status.data_ptr(), None)
    capi.call("hm_moe_layer_forward", C.byref(block.layer.desc), h.data_ptr(), gamma.data_ptr(),
              EPS, normed.data_ptr(), w.data_ptr(), T, block.top_k, block.flags | flags,
              block.limbs_x, block.limbs_z, C.byref(io), ws.data_ptr(), ws.numel(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert P == ids.numel()
    return normed.cpu().numpy(), ids.cpu().numpy().view(np.uint32), out.cpu().numpy()


@pytest.fixture(scope="module")
def layer_f32():
    payload, scale, zp = synth.expert_layer(93, 0, E, H, I, False)
    return DeviceExpertLayer(payload, scale, zp, H, I), payload


@pytest.mark.parametrize("T", [1, 5])
@pytest.mark.parametrize("offset", [0, 1])
def test_layer_forward_fp32(dev, layer_f32, T, offset):
    """FP32-weight layers through hm_moe_layer_forward.  With the normalised
    rows 16-byte aligned, decode batches take the FP32 GEMV and the result
    equals hm_rmsnorm followed by hm_moe_block_forward bit for bit; with
    them 4 bytes off, the call takes the FP32 tiles instead (the GEMV needs
    16-byte rows) rather than refusing.  Either way: the norm bit-exact, the
    routing bit-exact, the output within 1e-3 of the reference arithmetic."""
    import torch
    print(f"[gpu] FP32 layer forward T={T} normed offset={offset}", flush=True)
    dl, payload = layer_f32
    rng = np.random.default_rng(3000 + T)
    h = rng.standard_normal((T, H)).astype(np.float32)
    gamma = (0.5 + rng.random(H)).astype(np.float32)
    w = synth.router_weights(93, 0, H, E)
    dh, dg, dw = (torch.from_numpy(a).cuda() for a in (h, gamma, w))
    block = MoEBlock(dl, K)
    normed, ids, out = _layer_forward(block, dh, dg, dw, 0, normed_offset=offset)
    ref_norm = O.rmsnorm(h, gamma, EPS)
    assert_bitexact(normed, ref_norm, f"T={T} RMSNorm")
    ones = np.ones((E, 3), np.float32)
    zeros = np.zeros((E, 3), np.int32)
    rout, rids, _ = O.moe_block(payload, ones, zeros, ref_norm, w, K, I)
    assert_bitexact(ids, rids, f"T={T} routing vs oracle")
    moe = out - h  # the residual is added last, exactly
    err = float(np.abs(moe - rout).max() / np.abs(rout).max())
    assert err < 1e-3, f"T={T} offset={offset}: normwise error {err}"
    if offset == 0:
        dn = torch.empty_like(dh)
        capi.call("hm_rmsnorm", dh.data_ptr(), dg.data_ptr(), dn.data_ptr(), T, H, EPS,
                  torch.cuda.current_stream().cuda_stream)
        ref = block.execute_batch(dn, dw, residual=dh)
        assert_bitexact(ids, ref.ids, f"T={T} routing")
        assert_bitexact(out, ref.output.cpu().numpy(), f"T={T} output")


@pytest.mark.parametrize("T", [1, 2, 5, 16, 40])
@pytest.mark.parametrize("seq", [False, True])
def test_layer_forward_matches_norm_then_block(dev, layer, T, seq):
    import torch
    print(f"[gpu] layer forward T={T} seq={seq}", flush=True)
    rng = np.random.default_rng(1000 + T)
    row0, gamma, picked = _unsettled_row(rng, EPS)
    h = rng.standard_normal((T, H)).astype(np.float32)
    h[0] = row0
    w = synth.router_weights(91, 0, H, E)
    dh, dg, dw = (torch.from_numpy(a).cuda() for a in (h, gamma, w))
    block = MoEBlock(layer, K)
    flags = capi.HM_EXEC_ROUTE_SEQUENTIAL if seq else 0
    normed, ids, out = _layer_forward(block, dh, dg, dw, flags)
    # the normalised rows: the oracle's RMSNorm, bit for bit (row 0's
    # unsettled elements included)
    ref_norm = O.rmsnorm(h, gamma, EPS)
    assert_bitexact(normed, ref_norm, f"T={T} RMSNorm")
    assert_bitexact(normed[0, picked], ref_norm[0, picked], f"T={T} unsettled elements")
    # hm_rmsnorm on the device, then the block with h as the residual
    dn = torch.empty_like(dh)
    capi.call("hm_rmsnorm", dh.data_ptr(), dg.data_ptr(), dn.data_ptr(), T, H, EPS,
              torch.cuda.current_stream().cuda_stream)
    ref = block.execute_batch(dn, dw, residual=dh, exec_flags=flags)
    assert_bitexact(dn.cpu().numpy(), ref_norm, f"T={T} hm_rmsnorm")
    assert_bitexact(ids, ref.ids, f"T={T} routing")
    assert_bitexact(out, ref.output.cpu().numpy(), f"T={T} output")


def _sequential_sum_rows(rng, T, width):
    """Rows whose sequential sum of squares stresses its roundings: random
    rows, a tiny first element, leading zeros, magnitudes spread over 2^64
    that climb in every 256-element stretch (the sum changes binade over
    and over), odd integers after a 1.5 * 2^26 head (every step a tie,
    rounded to even), the same after a head just under 2^54 with occasional
    2^31-sized squares (ties next to a binade change), a log-normal row, all
    zeros, all ones (the sum reaches each power of two exactly), sparse
    powers of two and small odd multiples of powers of two."""
    k = np.arange(width)
    rows = np.empty((T, width), np.float32)
    for t in range(T):
        kind = t % 12
        if kind == 0:
            r = rng.standard_normal(width)
        elif kind == 1:
            r = rng.standard_normal(width)
            r[0] = 1e-20
        elif kind == 2:
            r = rng.standard_normal(width)
            r[:min(width - 1, 100 + int(rng.integers(200)))] = 0.0
        elif kind == 3:
            r = np.ldexp(1.0, (k % 256) // 4 - 32) * (1.0 + rng.random(width))
        elif kind == 4:
            r = (2 * rng.integers(0, 4, width) + 1).astype(np.float64)
            r[0] = 1.5 * 2.0 ** 26
        elif kind == 5:
            r = (2 * rng.integers(0, 4, width) + 1).astype(np.float64)
            big = rng.random(width) < 0.02
            r[big] = 46341 + 2 * rng.integers(0, 100, int(big.sum()))
            r[0] = 2.0 ** 27 - 8
        elif kind == 6:
            r = np.exp(rng.standard_normal(width) * 8.0)
        elif kind == 7:
            r = np.zeros(width)
        elif kind == 8:
            r = np.ones(width)
        elif kind == 9:
            r = np.where(rng.random(width) < 0.5, 0.0,
                         np.ldexp(1.0, rng.integers(-30, 30, width)))
        elif kind == 10:
            r = np.ldexp(rng.integers(1, 9, width).astype(np.float64), rng.integers(0, 6, width))
            r[:40] *= 4096.0
        else:
            r = np.ldexp((2 * rng.integers(0, 16, width) + 1).astype(np.float64),
                         rng.integers(-12, 12, width))
        rows[t] = r * np.where(rng.random(width) < 0.5, -1.0, 1.0)
    return rows


_WIDTH_LAYERS = {}


def _width_layer(width):
    if width == H:
        return None
    if width not in _WIDTH_LAYERS:
        payload, scale, zp = synth.expert_layer(95, 0, E, width, I, True)
        _WIDTH_LAYERS[width] = DeviceExpertLayer(payload, scale, zp, width, I)
    return _WIDTH_LAYERS[width]


@pytest.mark.parametrize("width,T,offset", [(H, 16, 0), (H, 24, 0), (H, 24, 1), (256, 24, 0),
                                            (768, 24, 0), (4096, 24, 0), (4096, 12, 0)])
def test_layer_forward_sequential_sum_rows(dev, layer, width, T, offset):
    """HM_EXEC_ROUTE_SEQUENTIAL sends every row of hm_moe_layer_forward to
    the sequential sum of squares: the decode fold in the router's first
    kernel (T <= 16), rmsnorm_wave_kernel (prefill, rows 16-byte aligned;
    widths of 1, 3, 8 and 16 times 256) and rmsnorm_kernel (normalised rows
    4 bytes off).  On rows built to stress that sum's roundings the
    normalised rows equal the oracle's RMSNorm bit for bit, and so do
    hm_rmsnorm's without the flag (the bracket, or the same fallback)."""
    import torch
    print(f"[gpu] sequential sum rows width={width} T={T} offset={offset}", flush=True)
    rng = np.random.default_rng(4000 + width + T + offset)
    dl = _width_layer(width) or layer
    h = _sequential_sum_rows(rng, T, width)
    gamma = (0.5 + rng.random(width)).astype(np.float32)
    w = synth.router_weights(95, 0, width, E)
    dh, dg, dw = (torch.from_numpy(a).cuda() for a in (h, gamma, w))
    block = MoEBlock(dl, K)
    normed, _, _ = _layer_forward(block, dh, dg, dw, capi.HM_EXEC_ROUTE_SEQUENTIAL,
                                  normed_offset=offset)
    ref = O.rmsnorm(h, gamma, EPS)
    assert np.isfinite(ref).all()
    for t in range(T):
        assert_bitexact(normed[t], ref[t], f"width={width} T={T} row {t} (kind {t % 12})")
    dn = torch.full_like(dh, float("nan"))
    capi.call("hm_rmsnorm", dh.data_ptr(), dg.data_ptr(), dn.data_ptr(), T, width, EPS,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert_bitexact(dn.cpu().numpy(), ref, f"width={width} T={T} hm_rmsnorm")


@pytest.mark.parametrize("T,offset", [(9, 0), (16, 0), (16, 1)])
def test_layer_forward_limb_decode(dev, layer, T, offset):
    """A decode batch of more than HM_GEMV_MAX_PAIRS pairs (top-8 here) takes
    the limb GEMMs; with the layer's RMSNorm folded into the router, the
    select kernel cuts the activation digits from the normalised rows (rows
    4 bytes off 16-byte alignment: the separate quantisation launch does):
    the same bits as hm_rmsnorm followed by the block."""
    import torch
    k = 8
    assert T * k > capi.HM_GEMV_MAX_PAIRS
    print(f"[gpu] layer forward limb decode T={T} offset={offset}", flush=True)
    rng = np.random.default_rng(2000 + T)
    row0, gamma, _ = _unsettled_row(rng, EPS)
    h = rng.standard_normal((T, H)).astype(np.float32)
    h[0] = row0
    w = synth.router_weights(91, 0, H, E)
    dh, dg, dw = (torch.from_numpy(a).cuda() for a in (h, gamma, w))
    block = MoEBlock(layer, k)
    normed, ids, out = _layer_forward(block, dh, dg, dw, 0, normed_offset=offset)
    assert_bitexact(normed, O.rmsnorm(h, gamma, EPS), f"T={T} RMSNorm")
    dn = torch.empty_like(dh)
    capi.call("hm_rmsnorm", dh.data_ptr(), dg.data_ptr(), dn.data_ptr(), T, H, EPS,
              torch.cuda.current_stream().cuda_stream)
    ref = block.execute_batch(dn, dw, residual=dh)
    assert_bitexact(ids, ref.ids, f"T={T} routing")
    assert_bitexact(out, ref.output.cpu().numpy(), f"T={T} output")


@pytest.mark.parametrize("T", [9, 13])
def test_rmsnorm_rows_unsettled_in_other_waves(dev, T):
    """hm_rmsnorm at H = 2048 runs one wave per row, four rows per
    workgroup: unsettled rows in wave slots 1 and 2 of different workgroups
    take the sequential sum on their own, the settled rows beside them do
    not, and the last workgroup's waves past the final row do nothing."""
    import torch
    print(f"[gpu] rmsnorm unsettled rows T={T}", flush=True)
    rng = np.random.default_rng(2000 + T)
    row0, gamma, picked = _unsettled_row(rng, EPS)
    h = rng.standard_normal((T, H)).astype(np.float32)
    h[1] = row0
    h[6] = row0
    dh, dg = torch.from_numpy(h).cuda(), torch.from_numpy(gamma).cuda()
    dn = torch.full_like(dh, float("nan"))
    capi.call("hm_rmsnorm", dh.data_ptr(), dg.data_ptr(), dn.data_ptr(), T, H, EPS,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = O.rmsnorm(h, gamma, EPS)
    got = dn.cpu().numpy()
    assert_bitexact(got, ref, f"T={T} hm_rmsnorm")
    for r in (1, 6):
        assert_bitexact(got[r, picked], ref[r, picked], f"T={T} row {r} unsettled elements")


def test_layer_forward_rejects_overlap(dev, layer):
    """normed overlapping h, or a residual other than h, is refused before
    anything runs."""
    import torch
    block = MoEBlock(layer, K)
    T = 2
    h = torch.randn((T, H), dtype=torch.float32, device="cuda")
    g = torch.ones(H, dtype=torch.float32, device="cuda")
    w = torch.from_numpy(synth.router_weights(91, 0, H, E)).cuda()
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    other = torch.empty((T, H), dtype=torch.float32, device="cuda")
    need = capi.load().hm_moe_block_workspace_bytes(C.byref(layer.desc), T, K, 2, 3, 0)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    lib = capi.load()
    s = torch.cuda.current_stream().cuda_stream
    for normed_ptr, residual in ((h.data_ptr() + 4 * H, None), (other.data_ptr(), out.data_ptr())):
        io = capi.HmBlockIO(out.data_ptr(), None, None, None, None, None, None, None, None,
                            residual)
        rc = lib.hm_moe_layer_forward(C.byref(layer.desc), h.data_ptr(), g.data_ptr(), EPS,
                                      normed_ptr, w.data_ptr(), T, K, 0, 2, 3, C.byref(io),
                                      ws.data_ptr(), ws.numel(), s)
        assert rc == capi.HM_ERR_INVALID
    torch.cuda.synchronize()
