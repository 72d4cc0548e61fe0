"""The synthetic-input generator (host/hm_synth.c) follows its documented
specification and is a sound N(mean, std) source.  CPU only."""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

import hm_oracle as O
from hmoe import synth


def test_splitmix_stream_matches_spec():
    lib = synth.load()
    for seed, tag in ((0, 0), (20240601, 1), (2 ** 63 + 5, 0x100 + 7)):
        key = lib.hm_synth_key(seed, tag)
        assert key == synth.spec_key(seed, tag)
        for i in (0, 1, 2, 1000, 2 ** 40):
            assert lib.hm_synth_u64(key, i) == synth.spec_u64(key, i)


def test_series_ln_and_cos_are_accurate():
    lib = synth.load()
    rng = np.random.default_rng(0)
    for u in np.concatenate([rng.random(2000), [2.0 ** -53, 1e-300, 0.5, 1.0, 0.70710678]]):
        u = float(u) if u > 0 else 2.0 ** -53
        assert abs(lib.hm_synth_ln(u) - math.log(u)) <= 4e-16 * max(1.0, abs(math.log(u)))
    c, s = C.c_double(), C.c_double()
    for u in np.concatenate([rng.random(2000), [0.0, 0.25, 0.5, 0.75, 0.999999]]):
        lib.hm_synth_cossin(float(u), C.byref(c), C.byref(s))
        assert abs(c.value - math.cos(2 * math.pi * u)) < 2e-15
        assert abs(s.value - math.sin(2 * math.pi * u)) < 2e-15


def test_normal_values_follow_box_muller():
    seed, tag = 11, 3
    vals = synth.normal(seed, tag, 64, 0.5, 2.0)
    for j in range(32):
        a, b = synth.spec_normal_pair(seed, tag, j, 0.5, 2.0)
        # same formula; series vs libm transcendentals differ by < 1e-15 rel
        assert abs(vals[2 * j] - a) <= 1e-6 * max(1.0, abs(a))
        assert abs(vals[2 * j + 1] - b) <= 1e-6 * max(1.0, abs(b))


def test_normal_statistics_and_determinism():
    x = synth.normal(1, 2, 400000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert np.array_equal(x, synth.normal(1, 2, 400000))
    assert not np.array_equal(x[:1000], synth.normal(1, 3, 1000))
    y = synth.normal(1, 2, 1001)
    assert np.array_equal(y[:1000], x[:1000]), "prefix property of the stream"


def test_layer_is_thread_count_independent():
    a = synth.expert_layer(5, 1, 3, 64, 32, True, threads=1)
    b = synth.expert_layer(5, 1, 3, 64, 32, True, threads=7)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    p, s, z = a
    assert p.shape == (3, 3, 64 * 32) and (z == 0).all() and (s > 0).all()


def test_zipf_skew_makes_a_hot_expert():
    """C4's routing skew (Zipf(1.1) ranking): on the C4 inputs the hottest
    expert gets about 10x the mean load and no expert is starved."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "oracle"))
    import hm_oracle as O
    cfg = synth.CONFIGS["C4"]
    T, H, E, k = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k
    h = O.rmsnorm(synth.raw_hidden(cfg.seed, T, H), np.ones(H, np.float32))
    w = synth.router_weights(cfg.seed, 0, H, E)
    synth.apply_skew(h, w, synth.zipf_bias(cfg.seed, E))
    rc, ids, sc = O.route(h, w, k, 1, 1)
    counts = np.bincount(ids.ravel(), minlength=E)
    assert 9.5 * counts.mean() <= counts.max() <= 10.5 * counts.mean()
    assert counts.min() > 0


def test_int8_payload_is_the_pinned_quantiser():
    """The generator's INT8 projections are the reference packer's symmetric
    quantisation (Quantization.cpp:45-79) of the float draws: every chosen
    projection regenerated from its tag and quantised by the oracle (and by
    the reference build where present) gives the payload bytes, scale and
    zero point bit for bit."""
    E, H, I = 3, 96, 64
    p, s, z = synth.expert_layer(5, 2, E, H, I, True, threads=2)
    for e in range(E):
        for proj in range(3):
            w = synth.normal(5, synth.tag_expert(2, e, proj), H * I, 0.0, 0.02)
            q, sc, zp, _ = O.quantize_int8(w)
            assert np.array_equal(q, p[e, proj]), (e, proj)
            assert np.float32(sc).view(np.uint32) == s[e, proj].view(np.uint32)
            assert zp == z[e, proj] == 0
            if O.ref_available():
                rq, rs, rz, _ = O.ref_quantize_int8(w)
                assert np.array_equal(rq, q) and rs == sc and rz == zp
