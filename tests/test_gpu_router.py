"""GPU parity: RMSNorm (A1), router top-k (A2), permute (A3), gather (A4),
combine (A7) and the expf boundary, against the CPU oracle (bit-exact)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact
from hmoe import synth

pytestmark = pytest.mark.gpu


def run_router(dev, h, w, k, flags):
    T, H = h.shape
    E = w.shape[1]
    ws = dev.empty(dev.lib.hm_route_workspace_bytes(T, H, E), np.uint8)
    ids = dev.empty((T, k), np.int32)
    scores = dev.empty((T, k), np.float32)
    logits = dev.empty((T, E), np.float32)
    status = dev.zeros(1, np.int32)
    dh, dw = dev.to(h), dev.to(w)
    dev.call("hm_router_topk", dh.data_ptr(), dw.data_ptr(), T, H, E, k, flags, ids.data_ptr(),
             scores.data_ptr(), logits.data_ptr(), status.data_ptr(), ws.data_ptr(), dev.stream)
    counts = dev.empty(E, np.int32)
    offsets = dev.empty(E + 1, np.int32)
    ptok = dev.empty(T * k, np.int32)
    pw = dev.empty(T * k, np.float32)
    slots = dev.empty(T * k, np.int32)
    st = int(dev.host(status)[0])
    if st == 0:
        pws = dev.empty(max(1, dev.lib.hm_permute_workspace_bytes(T, k, E)), np.uint8)
        dev.call("hm_permute", ids.data_ptr(), scores.data_ptr(), T, k, E, counts.data_ptr(),
                 offsets.data_ptr(), ptok.data_ptr(), pw.data_ptr(), slots.data_ptr(),
                 pws.data_ptr(), dev.stream)
    return dict(status=st, ids=dev.host(ids, np.uint32), scores=dev.host(scores),
                logits=dev.host(logits), counts=dev.host(counts), offsets=dev.host(offsets),
                ptok=dev.host(ptok), pw=dev.host(pw), slots=dev.host(slots).reshape(T, k))


CASES = [  # (T, H, E, k, softmax, renorm)
    (1, 2048, 128, 8, 1, 1), (4, 2048, 128, 8, 1, 1), (16, 2048, 64, 8, 1, 1),
    (33, 2048, 128, 8, 1, 1), (512, 2048, 64, 8, 1, 1), (7, 64, 3, 2, 1, 1),
    (9, 100, 130, 5, 1, 0), (9, 100, 200, 3, 0, 0), (9, 100, 200, 3, 0, 1),
    (65, 33, 1000, 64, 1, 1),
]


@pytest.mark.parametrize("T,H,E,k,sm,rn", CASES)
def test_router_and_permute_bitexact(dev, T, H, E, k, sm, rn):
    print(f"[gpu] router T={T} H={H} E={E} k={k} softmax={sm} renorm={rn}", flush=True)
    rng = np.random.default_rng(T * 1000 + E)
    h = O.rmsnorm(rng.standard_normal((T, H)).astype(np.float32), np.ones(H, np.float32))
    w = (0.02 * rng.standard_normal((H, E))).astype(np.float32)
    if not sm and rn:  # keep the raw-logit sum away from zero
        w = np.abs(w)
        h = np.abs(h)
    flags = (1 if sm else 0) | (2 if rn else 0)
    g = run_router(dev, h, w, k, flags)
    rc, logits = O.router_logits(h, w)
    assert rc == 0
    assert_bitexact(g["logits"], logits, "logits")
    rc, ids, scores = O.route(h, w, k, sm, rn)
    assert rc == 0 and g["status"] == 0
    assert_bitexact(g["ids"], ids, "top-k ids")
    assert_bitexact(g["scores"], scores, "scores")
    counts, offsets, ptok, pw, slots = O.group(ids, scores, E)
    assert_bitexact(g["counts"], counts, "counts")
    assert_bitexact(g["offsets"], offsets, "offsets")
    assert_bitexact(g["ptok"], ptok, "permutation")
    assert_bitexact(g["pw"], pw, "permuted weights")
    assert_bitexact(g["slots"], slots, "slots")


def test_router_reference_closed_forms(dev):
    """tests/phase7_tests.cpp:155-183 and phase8_tests.cpp:153-171."""
    h = np.array([[1.0, 0.0]], np.float32)
    w = np.array([[1, 3, 2], [0, 0, 0]], np.float32)
    g = run_router(dev, h, w, 2, 3)
    assert g["ids"].tolist() == [[1, 2]]
    assert abs(float(g["scores"].sum()) - 1.0) < 1e-6
    g = run_router(dev, h, w, 1, 0)
    assert g["ids"].tolist() == [[1]]
    w_tie = np.array([[1, 1, 1], [0, 0, 0]], np.float32)
    g = run_router(dev, h, w_tie, 2, 3)
    assert g["ids"].tolist() == [[0, 1]], "equal scores break ties by ascending expert id"
    hb = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    wb = np.array([[3, 2, 1], [0, 4, 1]], np.float32)
    g = run_router(dev, hb, wb, 2, 3)
    assert g["ids"][0].tolist() == [0, 1] and g["ids"][1].tolist() == [1, 2]
    # phase12_tests.cpp:269-273 grouping {0,2},{0,1,2},{1}
    h12 = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    w12 = np.array([[3, 2, 0], [0, 2, 3]], np.float32)
    g = run_router(dev, h12, w12, 2, 3)
    off = g["offsets"]
    groups = [g["ptok"][off[e]:off[e + 1]].tolist() for e in range(3)]
    assert groups == [[0, 2], [0, 1, 2], [1]]


@pytest.mark.parametrize("T", [2, 64])
def test_router_wide_spread_uses_sequential_denominator(dev, T):
    """Logits spread > 12: some softmax terms fall below 2^-17, so the select
    kernel takes its sequential double-sum path (T = 2: the one-workgroup
    select, every thread on one token)."""
    rng = np.random.default_rng(5)
    H, E, k = 256, 128, 8
    h = O.rmsnorm(rng.standard_normal((T, H)).astype(np.float32), np.ones(H, np.float32))
    w = (1.5 * rng.standard_normal((H, E))).astype(np.float32)
    g = run_router(dev, h, w, k, 3)
    rc, ids, scores = O.route(h, w, k, 1, 1)
    assert rc == 0
    assert_bitexact(g["ids"], ids, "ids")
    assert_bitexact(g["scores"], scores, "scores")


@pytest.mark.parametrize("T", [3, 40])
def test_router_ties_and_duplicates(dev, T):
    """Many exactly equal logits (duplicated router columns): ranks by key
    (T = 3) and rounds of argmax (T = 40) break ties by ascending id."""
    rng = np.random.default_rng(9)
    H, E, k = 64, 64, 8
    h = rng.standard_normal((T, H)).astype(np.float32)
    base = (0.02 * rng.standard_normal((H, 8))).astype(np.float32)
    w = np.tile(base, (1, E // 8))
    for flags, sm, rn in ((3, 1, 1), (0, 0, 0)):
        g = run_router(dev, h, w, k, flags)
        rc, ids, scores = O.route(h, w, k, sm, rn)
        assert_bitexact(g["ids"], ids, "ids with ties")
        assert_bitexact(g["scores"], scores, "scores with ties")


def test_router_nonfinite_sets_status(dev):
    """CpuRouterBackend.cpp:47 throws on a non-finite score; the device sets
    HM_STATUS_NONFINITE_SCORE."""
    h = np.array([[1.0, 2.0]], np.float32)
    w = np.array([[np.inf, 1.0], [0.0, 0.0]], np.float32)
    g = run_router(dev, h, w, 1, 3)
    assert g["status"] & 1
    # a failed token still gets in-range placeholder ids for the stages after it
    assert (g["ids"] < 2).all()
    rc, _, _ = O.route(h, w, 1, 1, 1)
    assert rc == -3  # HMO_E_RUNTIME


def test_router_sequential_flag_same_bits(dev):
    """Decode batches certify parallel block sums of the logits, prefill
    batches FP64 matrix-core sums; forcing the reference's sequential chain
    for every logit gives the same bits."""
    from hmoe import capi
    # (H = 96, 160: the chains' last 64-product piece is a half one)
    for T, H, E in ((1, 2048, 128), (16, 2048, 128), (5, 512, 64), (40, 2048, 128),
                    (300, 2048, 128), (100, 512, 64), (70, 64, 192), (5, 96, 64),
                    (1, 160, 128)):
        print(f"[gpu] router sequential flag T={T} H={H} E={E}", flush=True)
        rng = np.random.default_rng(T + H)
        h = O.rmsnorm(rng.standard_normal((T, H)).astype(np.float32), np.ones(H, np.float32))
        w = (0.02 * rng.standard_normal((H, E))).astype(np.float32)
        a = run_router(dev, h, w, 8, 3)
        b = run_router(dev, h, w, 8, 3 | capi.HM_EXEC_ROUTE_SEQUENTIAL)
        rc, logits = O.router_logits(h, w)
        assert_bitexact(a["logits"], logits, "certified logits")
        assert_bitexact(b["logits"], logits, "sequential logits")
        assert_bitexact(a["ids"], b["ids"], "ids")
        assert_bitexact(a["scores"], b["scores"], "scores")


@pytest.mark.parametrize("T,E", [(2, 4), (2, 64), (40, 64)])
def test_router_uncertifiable_logits(dev, T, E):
    """Logits the bound cannot settle fall back to the sequential chain:
    an exact float midpoint (1 + 2^-24 ties to even: 1.0) and an exact
    cancellation (the sequential sum ends at +0, the interval spans -0/+0).
    T = 2: decode block sums; T = 40, E = 64: matrix-core sums."""
    H = 64
    rng = np.random.default_rng(T + E)
    h = np.zeros((T, H), np.float32)
    w = np.zeros((H, E), np.float32)
    h[2:] = rng.standard_normal((T - 2, H)).astype(np.float32)
    w[:, 4:] = (0.02 * rng.standard_normal((H, E - 4))).astype(np.float32)
    h[0, 0], h[0, 1] = 1.0, 2.0 ** -24
    w[0, :], w[1, :] = 1.0, 1.0            # expert logits 1 + 2^-24 -> 1.0
    h[1, 0], h[1, 5] = 1.0, 1.0
    w[0, 2], w[5, 2] = 0.375, -0.375       # expert 2 of token 1: exactly 0
    w[0, 3], w[5, 3] = 3.0, 2.0 ** -22     # expert 3 of token 1: 3 + 2^-22 (exact)
    g = run_router(dev, h, w, 2, 3)
    rc, logits = O.router_logits(h, w)
    assert rc == 0
    assert_bitexact(g["logits"], logits, "logits at rounding boundaries")
    assert g["logits"][0, 0] == 1.0
    assert np.signbit(g["logits"][1, 2]) == np.signbit(logits[1, 2]) and g["logits"][1, 2] == 0.0
    rc, ids, scores = O.route(h, w, 2, 1, 1)
    assert_bitexact(g["ids"], ids, "ids")
    assert_bitexact(g["scores"], scores, "scores")


@pytest.mark.parametrize("T,E", [(1, 8), (1, 64), (20, 64)])
def test_router_parallel_nonfinite_sets_status(dev, T, E):
    """A non-finite logit on the certified paths (it always takes the
    sequential chain) sets HM_STATUS_NONFINITE_SCORE."""
    H = 64
    h = np.ones((T, H), np.float32)
    w = np.full((H, E), 0.01, np.float32)
    w[3, 5] = np.inf
    g = run_router(dev, h, w, 2, 3)
    assert g["status"] & 1
    assert (g["ids"] < E).all()


def test_permute_invariants_large(dev):
    """C4 shape (T=4096, E=128, k=8) with Zipf-skewed routing: permutation
    bit-exact against the oracle grouping of the oracle's routing."""
    cfg = synth.CONFIGS["C4"]
    T, H, E, k = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k
    h = O.rmsnorm(synth.raw_hidden(cfg.seed, T, H), np.ones(H, np.float32))
    w = synth.router_weights(cfg.seed, 0, H, E)
    synth.apply_skew(h, w, synth.zipf_bias(cfg.seed, E))
    g = run_router(dev, h, w, k, 3)
    rc, ids, scores = O.route(h, w, k, 1, 1)
    assert rc == 0
    assert_bitexact(g["ids"], ids, "ids")
    assert_bitexact(g["scores"], scores, "scores")
    counts, offsets, ptok, pw, slots = O.group(ids, scores, E)
    assert_bitexact(g["ptok"], ptok, "permutation")
    assert g["counts"].sum() == T * k
    assert g["counts"].max() >= 5 * T * k / E, "Zipf skew should make a hot expert"


@pytest.mark.parametrize("rows,width", [(1, 2048), (3, 2), (64, 2048), (300, 777)])
def test_rmsnorm_bitexact(dev, rows, width):
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal((rows, width)) * rng.uniform(0.01, 100, (rows, 1))).astype(np.float32)
    g = rng.uniform(0.5, 2, width).astype(np.float32)
    y = dev.empty((rows, width), np.float32)
    dev.call("hm_rmsnorm", dev.to(x).data_ptr(), dev.to(g).data_ptr(), y.data_ptr(), rows, width,
             1e-6, dev.stream)
    assert_bitexact(dev.host(y), O.rmsnorm(x, g, 1e-6), "rmsnorm")


def test_rmsnorm_closed_form(dev):
    """tests/phase12_tests.cpp:182-198: [3,4],[0,2] with gamma [1,2]."""
    x = np.array([[3, 4], [0, 2]], np.float32)
    g = np.array([1, 2], np.float32)
    y = dev.empty((2, 2), np.float32)
    dev.call("hm_rmsnorm", dev.to(x).data_ptr(), dev.to(g).data_ptr(), y.data_ptr(), 2, 2, 1e-6,
             dev.stream)
    a = np.float32(1.0 / np.sqrt(12.5 + 1e-6))
    b = np.float32(1.0 / np.sqrt(2.0 + 1e-6))
    np.testing.assert_allclose(dev.host(y), [[3 * a, 8 * a], [0, 4 * b]], rtol=1e-6)


def test_device_expf_matches_libm(dev):
    """The libm boundary: device expf vs host glibc expf, bit-exact, on a
    stride through all float bit patterns plus edge values."""
    pats = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)
    x = pats.view(np.float32)
    x = x[np.isfinite(x)]
    x = np.concatenate([x, np.array([0.0, -0.0, 88.0, 88.72283, 88.72284, -103.97,
                                     -103.973, -104.0, -np.inf, np.inf], np.float32)])
    y = dev.empty(x.shape, np.float32)
    dev.call("hm_debug_expf", dev.to(x).data_ptr(), y.data_ptr(), x.size, dev.stream)
    libm = C.CDLL("libm.so.6")
    libm.expf.restype = C.c_float
    libm.expf.argtypes = [C.c_float]
    sample = np.arange(0, x.size, max(1, x.size // 200000))
    got = dev.host(y)[sample]
    ref = np.array([libm.expf(float(v)) for v in x[sample]], np.float32)
    assert_bitexact(got, ref, "device expf vs libm expf")


def test_gather_and_combine_closed_form(dev):
    """tests/phase18_19_tests.cpp:251-263: gather rows {2,0}, weights
    {0.5, 2} -> [-4,-2,0,0,1,1.5]."""
    x = np.array([[-2, -1], [0, 1], [2, 3]], np.float32)
    rows = np.array([2, 0], np.int32)
    out = dev.empty((2, 2), np.float32)
    dev.call("hm_gather_rows", dev.to(x).data_ptr(), dev.to(rows).data_ptr(), 2, 2,
             out.data_ptr(), dev.stream)
    g = dev.host(out)
    assert g.tolist() == [[2, 3], [-2, -1]]
    # combine: token 2 <- row 0 (w 0.5), token 0 <- row 1 (w 2); top_k = 1
    ids = np.array([[1], [0], [0]], np.uint32)
    slots = np.array([[1], [0], [0]], np.int32)
    scores = np.array([[2.0], [0.0], [0.5]], np.float32)
    y = np.array([[2, 3], [-2, -1]], np.float32)
    res = dev.empty((3, 2), np.float32)
    dev.call("hm_combine", dev.to(y).data_ptr(), dev.to(ids).data_ptr(), dev.to(slots).data_ptr(),
             dev.to(scores).data_ptr(), 3, 1, 2, None, res.data_ptr(), dev.stream)
    r = dev.host(res)
    assert r[0].tolist() == [-4, -2] and r[2].tolist() == [1, 1.5]
