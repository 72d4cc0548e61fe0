"""The packed-artefact loader (include/hm_artefact.hpp, host/artefact.cpp):
the reference's experts.index / manifest.json / experts.bin formats,
their validation, CRC32, and the layer it hands to the device.

Format parity is pinned against the compiled reference where it is built
(oracle/_ref: storage::ExpertIndex::save/load, storage::ExpertStore::crc32,
models::ModelManifest::load + validate): the reference writes byte-identical
index files, reads this build's files to the same records, accepts this
build's manifests, and rejects the same malformed files.  CRC32 is also
pinned by its published check value (CRC-32/ISO-HDLC of "123456789")."""
from __future__ import annotations

import ctypes as C
import json
import struct
import zlib

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact, assert_compare
from hmoe import artefact as A
from hmoe import capi
from hmoe import synth

HAVE_REF = O.ref_available()
needs_ref = pytest.mark.skipif(not HAVE_REF, reason="reference build not present")


def _ref():
    lib = O.ref()
    lib.hmref_crc32.restype, lib.hmref_crc32.argtypes = C.c_uint32, [C.c_void_p, C.c_size_t]
    lib.hmref_index_save.restype = C.c_int
    lib.hmref_index_save.argtypes = [C.c_char_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    lib.hmref_index_load.restype = C.c_int
    lib.hmref_index_load.argtypes = [C.c_char_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t,
                                     C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    lib.hmref_manifest_load.restype = C.c_int
    lib.hmref_manifest_load.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    return lib


def _flat_records(records, projections):
    r = np.array([list(x) for x in records], np.uint64).reshape(-1, 6)
    p = np.array([list(x[:8]) + list(x[8]) + [x[9], x[10], 0, 0] for x in projections],
                 np.uint64).reshape(-1, 16)
    return np.ascontiguousarray(r), np.ascontiguousarray(p)


def ref_index_save(path, records, projections) -> int:
    r, p = _flat_records(records, projections)
    return _ref().hmref_index_save(str(path).encode(), r.ctypes.data, len(records),
                                   p.ctypes.data, len(projections))


def ref_index_load(path):
    lib = _ref()
    nr, np_ = C.c_size_t(), C.c_size_t()
    rc = lib.hmref_index_load(str(path).encode(), None, 0, None, 0, C.byref(nr), C.byref(np_))
    if rc:
        return rc, None, None
    r = np.zeros((max(1, nr.value), 6), np.uint64)
    p = np.zeros((max(1, np_.value), 16), np.uint64)
    rc = lib.hmref_index_load(str(path).encode(), r.ctypes.data, nr.value, p.ctypes.data,
                              np_.value, C.byref(nr), C.byref(np_))
    recs = [tuple(int(v) for v in x) for x in r[:nr.value]]
    projs = [tuple(int(v) for v in x[:8]) + (tuple(int(v) for v in x[8:12]), int(x[12]),
                                            int(x[13])) for x in p[:np_.value]]
    return rc, recs, projs


def ref_manifest(path):
    buf = C.create_string_buffer(1 << 22)
    rc = _ref().hmref_manifest_load(str(path).encode(), buf, len(buf))
    return rc, (json.loads(buf.value.decode()) if rc == 0 else None)


def small_records():
    recs = [(0, 0, 0, 6144, 6, 0x1234), (0, 1, 8192, 6144, 6, 0x5678),
            (1, 0, 16384, 8192, 0, 0xdeadbeef)]
    projs = [(0, 0, 0, 3, 2, 0, 0, 2048, (64, 32, 0, 0), 11, 0),
             (0, 0, 1, 3, 2, 0, 2048, 2048, (64, 32, 0, 0), 12, 0),
             (0, 0, 2, 3, 2, 0, 4096, 2048, (32, 64, 0, 0), 13, 0),
             (1, 0, 2, 0, 2, 0, 16384, 8192, (32, 64, 0, 0), 14, 0)]
    return recs, projs


def test_crc32_check_value_and_zlib():
    """CRC-32/ISO-HDLC check value 0xCBF43926; equal to zlib's CRC-32."""
    assert A.crc32(b"123456789") == 0xCBF43926
    rng = np.random.default_rng(0)
    for n in (0, 1, 7, 4096, 100001):
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert A.crc32(b) == zlib.crc32(b)


@needs_ref
def test_crc32_equals_reference_store():
    rng = np.random.default_rng(1)
    for n in (0, 3, 1000, 65537):
        b = rng.integers(0, 256, n, dtype=np.uint8)
        assert A.crc32(b) == _ref().hmref_crc32(b.ctypes.data, n)


def test_index_round_trip(tmp_path):
    recs, projs = small_records()
    for v, (r, p) in ((2, (recs, projs)), (1, (recs, []))):
        path = tmp_path / f"v{v}.index"
        A.write_index(path, r, p)
        raw = path.read_bytes()
        assert raw[:8] == b"HMOEIDX\0" and struct.unpack_from("<I", raw, 8)[0] == v
        r2, p2 = A.read_index(path)
        assert r2 == r and p2 == p


@needs_ref
def test_index_bytes_equal_reference_writer(tmp_path):
    """The reference's ExpertIndex::save writes the same bytes, and its
    ExpertIndex::load reads this build's file to the same records."""
    recs, projs = small_records()
    for r, p in ((recs, projs), (recs, [])):
        ours, theirs = tmp_path / "ours.index", tmp_path / "ref.index"
        A.write_index(ours, r, p)
        assert ref_index_save(theirs, r, p) == 0
        assert ours.read_bytes() == theirs.read_bytes()
        rc, r2, p2 = ref_index_load(ours)
        assert rc == 0 and r2 == r and p2 == p


def _corruptions(raw: bytes):
    """Malformed variants of a valid v2 index image (name, bytes)."""
    b = bytearray(raw)
    out = []

    def mut(name, off, fmt, val):
        c = bytearray(b)
        struct.pack_into(fmt, c, off, val)
        out.append((name, bytes(c)))

    mut("magic", 0, "<B", ord("X"))
    mut("version", 8, "<I", 3)
    mut("endian", 12, "<I", 0x04030201)
    mut("record size", 16, "<I", 31)
    mut("extension size", 20, "<I", 0)
    mut("record count", 24, "<Q", 4)
    out.append(("truncated", bytes(b[:-1])))
    out.append(("trailing data", bytes(b) + b"\0"))
    rec0 = 32
    mut("zero size", rec0 + 16, "<Q", 0)
    mut("quantization code", rec0 + 24, "<I", 8)
    mut("duplicate key", rec0 + 32 + 4, "<I", 0)  # record 1 -> (0, 0)
    proj0 = 32 + 3 * 32 + 8
    mut("projection type", proj0 + 8, "<I", 3)
    mut("projection dtype", proj0 + 12, "<I", 4)
    mut("projection rank", proj0 + 16, "<I", 0)
    mut("projection reserved", proj0 + 20, "<I", 1)
    mut("projection escapes", proj0 + 24, "<Q", 6000)
    mut("projection size", proj0 + 32, "<Q", 2047)
    mut("zero dimension", proj0 + 40, "<Q", 0)
    mut("dimension beyond rank", proj0 + 56, "<Q", 1)
    mut("trailing reserved", proj0 + 76, "<I", 1)
    mut("duplicate projection", proj0 + 80 + 8, "<I", 0)
    return out


def test_index_rejects_malformed(tmp_path):
    recs, projs = small_records()
    good = tmp_path / "good.index"
    A.write_index(good, recs, projs)
    for name, data in _corruptions(good.read_bytes()):
        path = tmp_path / "bad.index"
        path.write_bytes(data)
        with pytest.raises(A.StorageError):
            A.read_index(path)
        if HAVE_REF:
            rc, _, _ = ref_index_load(path)
            assert rc != 0, f"the reference accepts the '{name}' case"


def _model(tmp_path, int8=True, layers=2, E=4, H=64, I=32, k=2, seed=5):
    out = []
    for l in range(layers):
        p, s, z = synth.expert_layer(seed, l, E, H, I, int8)
        per = A.layers_from_payload(p, s if int8 else None, z if int8 else None, E, H, I)
        out.append((per, synth.router_weights(seed, l, H, E)))
    d = tmp_path / "model"
    A.write_packed_model(d, out, H, I, k)
    return d, out


def test_packed_model_round_trip(tmp_path):
    d, layers = _model(tmp_path)
    m = A.PackedModel(d)
    assert (m.layers, m.experts, m.hidden, m.intermediate, m.top_k) == (2, 4, 64, 32, 2)
    assert m.dtype == 3 and m.route_flags == 3
    for l in range(2):
        p, s, z = m.read_layer(l)
        p0, s0, z0 = synth.expert_layer(5, l, 4, 64, 32, True)
        assert_bitexact(p, p0, "payload")
        assert_bitexact(s, s0, "scales")
        assert_bitexact(z, z0, "zero points")
        assert_bitexact(m.read_router(l), synth.router_weights(5, l, 64, 4), "router")
    recs, projs = A.read_index(d / "experts.index")
    assert all(r[2] % A.ALIGN == 0 for r in recs), "payloads are 4 KiB aligned"
    assert len(projs) == 3 * len(recs)


def test_packed_model_fp32_and_widened_16_bit(tmp_path):
    d, _ = _model(tmp_path, int8=False)
    m = A.PackedModel(d)
    p, _, _ = m.read_layer(1)
    assert m.dtype == 0 and p.dtype == np.float32
    assert_bitexact(p, synth.expert_layer(5, 1, 4, 64, 32, False)[0], "fp32 payload")
    for np_dtype, name in ((np.float16, "fp16"), (None, "bf16")):
        sub = tmp_path / name
        sub.mkdir()
        p0 = synth.expert_layer(5, 0, 4, 64, 32, False)[0]
        if np_dtype is not None:
            stored = p0.astype(np_dtype)
            expect = stored.astype(np.float32)
        else:
            stored = (p0.view(np.uint32) >> 16).astype(np.uint16)  # truncated bf16 bits
            expect = (stored.astype(np.uint32) << 16).view(np.float32)
        per = A.layers_from_payload(stored, None, None, 4, 64, 32)
        A.write_packed_model(sub, [(per, synth.router_weights(5, 0, 64, 4))], 64, 32, 2)
        got, _, _ = A.PackedModel(sub).read_layer(0)
        assert got.dtype == np.float32
        assert_bitexact(got, expect.reshape(got.shape), f"{name} widened to fp32")


@needs_ref
def test_reference_accepts_written_model(tmp_path):
    """models::ModelManifest::load (with validate) and ExpertIndex::load accept
    the written artefact and read the same model."""
    d, _ = _model(tmp_path)
    rc, canon = ref_manifest(d / "manifest.json")
    assert rc == 0
    ours = json.loads((d / "manifest.json").read_text())
    for key in ("schema", "layer_count", "expert_count", "hidden_size", "intermediate_size"):
        assert canon[key] == ours[key]
    assert canon["router"]["top_k"] == 2 and canon["router"]["tensors"] == ours["router"]["tensors"]
    assert [t["name"] for t in canon["tensors"]] == [t["name"] for t in ours["tensors"]]
    for a, b in zip(canon["tensors"], ours["tensors"]):
        assert (a["offset"], a["size"], a["shape"], a["dtype"]) == \
            (b["offset"], b["size"], b["shape"], b["dtype"])
        if "quantization" in b:
            assert np.float32(a["quantization"]["scale"]) == np.float32(b["quantization"]["scale"])
    assert canon["experts"] == ours["experts"]
    rc, recs, projs = ref_index_load(d / "experts.index")
    assert rc == 0 and (recs, projs) == A.read_index(d / "experts.index")


def test_checksums_detect_corruption(tmp_path):
    d, _ = _model(tmp_path)
    recs, _ = A.read_index(d / "experts.index")
    off = recs[5][2] + 100  # inside layer 1, expert 1
    raw = bytearray((d / "experts.bin").read_bytes())
    raw[off] ^= 0xFF
    (d / "experts.bin").write_bytes(bytes(raw))
    m = A.PackedModel(d)
    m.read_layer(0)  # untouched layer
    with pytest.raises(A.StorageError, match="checksum"):
        m.read_layer(1)
    A.PackedModel(d, verify_checksums=False).read_layer(1)


@pytest.mark.parametrize("edit", ["schema", "expert_count", "int8_without_quantization",
                                  "router_shape", "missing_expert", "projection_escapes"])
def test_manifest_rejects_inconsistent(tmp_path, edit):
    d, _ = _model(tmp_path)
    path = d / "manifest.json"
    m = json.loads(path.read_text())
    if edit == "schema":
        m["schema"] = "hypermoe.model-manifest.v9"
    elif edit == "expert_count":
        m["router"]["expert_count"] = 5
    elif edit == "int8_without_quantization":
        del m["tensors"][0]["quantization"]
    elif edit == "router_shape":
        rt = next(t for t in m["tensors"] if t["name"].endswith("router"))
        rt["shape"] = rt["shape"][::-1]
    elif edit == "missing_expert":
        m["experts"] = m["experts"][1:]
    elif edit == "projection_escapes":
        m["experts"][0]["gate"]["offset"] += 1
    path.write_text(json.dumps(m))
    with pytest.raises(ValueError):
        A.PackedModel(d)
    if HAVE_REF:
        assert ref_manifest(path)[0] != 0, "the reference accepts it"


@pytest.mark.gpu
def test_loaded_layer_runs_like_the_generated_one(tmp_path, dev):
    """A layer loaded from the artefact gives the same block results, bit for
    bit, as the same layer uploaded straight from the generator."""
    import torch
    from hmoe.block import DeviceExpertLayer, MoEBlock
    E, H, I, k = 16, 512, 256, 4
    d, _ = _model(tmp_path, E=E, H=H, I=I, k=k, layers=1, seed=9)
    m = A.PackedModel(d)
    layer, w = m.load_layer(0)
    p, s, z = synth.expert_layer(9, 0, E, H, I, True)
    ref_layer = DeviceExpertLayer(p, s, z, H, I)
    w0 = torch.from_numpy(synth.router_weights(9, 0, H, E)).cuda()
    for T in (3, 40):
        print(f"[gpu] artefact layer T={T}", flush=True)
        rng = np.random.default_rng(T)
        h = torch.from_numpy(O.rmsnorm(rng.standard_normal((T, H)).astype(np.float32),
                                       np.ones(H, np.float32))).cuda()
        a = MoEBlock(layer, m.top_k).execute_batch(h, w)
        b = MoEBlock(ref_layer, k).execute_batch(h, w0)
        assert_bitexact(a.ids, b.ids, "ids")
        assert_bitexact(a.output.cpu().numpy(), b.output.cpu().numpy(), "outputs")
        # and the loaded layer against the oracles: the reference block
        # (ids bit-exact, output within 1e-4) and, on the integer-limb path,
        # the limb restatement bit for bit
        hn, wn = h.cpu().numpy(), w0.cpu().numpy()
        rout, rids, _ = O.moe_block(p, s, z, hn, wn, k, I)
        assert_bitexact(a.ids, rids, "ids vs reference")
        assert_compare(a.output.cpu().numpy(), rout, 1e-4, 1e-4, "loaded layer vs reference block")
        la = MoEBlock(layer, m.top_k, limbs_x=2, limbs_z=3).execute_batch(
            h, w, exec_flags=capi.HM_EXEC_LIMBS)
        lout, _, _ = O.moe_block_limbs(p, s, z, hn, wn, k, I, 2, 3)
        assert_bitexact(la.output.cpu().numpy(), lout, "loaded layer vs limb oracle")


def test_host_library_exports_the_artefact_abi():
    import re
    from pathlib import Path
    header = Path(__file__).resolve().parent.parent / "include" / "hm_artefact.h"
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(hm_[a-z0-9_]+)\s*\(", text)))
    assert len(names) >= 8
    lib = A.load()
    assert [n for n in names if not hasattr(lib, n)] == []
    assert set(names) == set(A._SIGS)
