"""The reference's packed model artefact: ctypes binding of the loader in
libhm_host.so (include/hm_artefact.h), and a writer of the same format.

A packed model directory holds experts.bin, experts.index (v2) and
manifest.json (hypermoe.model-manifest.v3), as the reference's ExpertPacker
writes them (tools/model_convert/ExpertPacker.cpp:150-280): each expert's
payload 4 KiB aligned, gate | up | down back to back, [K x N] row-major
INPUT_OUTPUT, INT8 with one per-projection {scale, zero_point} in the
manifest or FP32; the routers' [H x E] FP32 matrices after the experts.

`PackedModel.load_layer` reads one layer (checking every expert's and
projection's CRC32) and uploads it as a DeviceExpertLayer with its router
matrix on the device.  `write_packed_model` writes the format (used by the
tests and to turn synthetic layers into an artefact).
"""
from __future__ import annotations

import ctypes as C
import json
import zlib
from pathlib import Path

import numpy as np

from . import build as _build
from . import capi

HM_ERR_STORAGE = 5
ALIGN = 4096  # ExpertPacker.cpp:23
QUANT_FP32, QUANT_INT8 = 0, 6  # QuantizationType (include/hypermoe/experts/expert.hpp:14-23)
DTYPE_CODE = {"FP32": 0, "FP16": 1, "BF16": 2, "INT8": 3}


class IndexRecord(C.Structure):
    _fields_ = [("layer_id", C.c_uint32), ("expert_id", C.c_uint32), ("offset", C.c_uint64),
                ("size", C.c_uint64), ("quantization_type", C.c_uint32), ("checksum", C.c_uint32)]


class ProjectionRecord(C.Structure):
    _fields_ = [("layer_id", C.c_uint32), ("expert_id", C.c_uint32),
                ("projection_type", C.c_uint32), ("dtype", C.c_uint32), ("rank", C.c_uint32),
                ("reserved", C.c_uint32), ("offset", C.c_uint64), ("size", C.c_uint64),
                ("shape", C.c_uint64 * 4), ("checksum", C.c_uint32),
                ("trailing_reserved", C.c_uint32)]


class PackedInfo(C.Structure):
    _fields_ = [("layers", C.c_uint32), ("experts", C.c_uint32), ("hidden", C.c_uint64),
                ("intermediate", C.c_uint64), ("dtype", C.c_uint32), ("top_k", C.c_uint32),
                ("route_flags", C.c_uint32)]


_SIGS = {
    "hm_artefact_last_error": (C.c_char_p, []),
    "hm_crc32": (C.c_uint32, [C.c_void_p, C.c_size_t]),
    "hm_index_read": (C.c_int32, [C.c_char_p, C.POINTER(IndexRecord), C.c_size_t,
                                  C.POINTER(ProjectionRecord), C.c_size_t,
                                  C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "hm_index_write": (C.c_int32, [C.c_char_p, C.POINTER(IndexRecord), C.c_size_t,
                                   C.POINTER(ProjectionRecord), C.c_size_t]),
    "hm_packed_open": (C.c_int32, [C.c_char_p, C.c_int32, C.POINTER(C.c_void_p)]),
    "hm_packed_close": (None, [C.c_void_p]),
    "hm_packed_info": (C.c_int32, [C.c_void_p, C.POINTER(PackedInfo)]),
    "hm_packed_read_layer": (C.c_int32, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_size_t,
                                         C.c_void_p, C.c_void_p]),
    "hm_packed_read_router": (C.c_int32, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_size_t]),
}

_lib = None


class StorageError(RuntimeError):
    """The reference's storage::StorageError (malformed index, missing or
    corrupt payload)."""


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not _build.HOST_SO.exists():
            raise RuntimeError(f"{_build.HOST_SO} is not built: run __graft_entry__.build()")
        lib = C.CDLL(str(_build.HOST_SO))
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    return _lib


def _check(rc: int) -> None:
    if rc == 0:
        return
    msg = load().hm_artefact_last_error().decode()
    if rc == HM_ERR_STORAGE:
        raise StorageError(msg)
    if rc == capi.HM_ERR_OVERFLOW:
        raise OverflowError(msg)
    if rc == capi.HM_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(f"{msg} (status {rc})")


def crc32(data: bytes | np.ndarray) -> int:
    b = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, bytes) else data)
    return int(load().hm_crc32(b.ctypes.data, b.nbytes))


def read_index(path) -> tuple[list[tuple], list[tuple]]:
    """ExpertIndex::load: (records, projections) as tuples in field order."""
    lib = load()
    nr, np_ = C.c_size_t(), C.c_size_t()
    _check(lib.hm_index_read(str(path).encode(), None, 0, None, 0, C.byref(nr), C.byref(np_)))
    recs = (IndexRecord * max(1, nr.value))()
    projs = (ProjectionRecord * max(1, np_.value))()
    _check(lib.hm_index_read(str(path).encode(), recs, nr.value, projs, np_.value, C.byref(nr),
                             C.byref(np_)))
    r = [(x.layer_id, x.expert_id, x.offset, x.size, x.quantization_type, x.checksum)
         for x in recs[:nr.value]]
    p = [(x.layer_id, x.expert_id, x.projection_type, x.dtype, x.rank, x.reserved, x.offset,
          x.size, tuple(x.shape), x.checksum, x.trailing_reserved) for x in projs[:np_.value]]
    return r, p


def write_index(path, records: list[tuple], projections: list[tuple]) -> None:
    """ExpertIndex(records, projections).save (v2 when there are projection
    records, else v1); raises on records the reference rejects."""
    rs = (IndexRecord * max(1, len(records)))(*[IndexRecord(*r) for r in records])
    ps = (ProjectionRecord * max(1, len(projections)))()
    for i, p in enumerate(projections):
        ps[i] = ProjectionRecord(*p[:8], (C.c_uint64 * 4)(*p[8]), p[9], p[10])
    _check(load().hm_index_write(str(path).encode(), rs, len(records), ps, len(projections)))


class PackedModel:
    """An opened packed model directory (host side: index, manifest and a
    read-only mapping of experts.bin)."""

    def __init__(self, directory, verify_checksums: bool = True):
        h = C.c_void_p()
        _check(load().hm_packed_open(str(directory).encode(), int(verify_checksums), C.byref(h)))
        self._h = h
        info = PackedInfo()
        _check(load().hm_packed_info(h, C.byref(info)))
        self.layers, self.experts = info.layers, info.experts
        self.hidden, self.intermediate = info.hidden, info.intermediate
        self.dtype, self.top_k, self.route_flags = info.dtype, info.top_k, info.route_flags

    def close(self) -> None:
        if self._h:
            load().hm_packed_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass

    def read_layer(self, layer: int):
        """(payload [E, 3, H*I] int8 or float32 in the synthetic generator's
        layout, scale [E, 3] float32, zero_point [E, 3] int32) of one layer,
        CRC-checked."""
        E, H, I = self.experts, self.hidden, self.intermediate
        width = 1 if self.dtype == capi.HM_DTYPE_INT8 else 4
        payload = np.empty(E * 3 * H * I * width, np.uint8)
        scale = np.empty((E, 3), np.float32)
        zp = np.empty((E, 3), np.int32)
        _check(load().hm_packed_read_layer(self._h, layer, payload.ctypes.data, payload.nbytes,
                                           scale.ctypes.data, zp.ctypes.data))
        payload = payload.view(np.int8 if self.dtype == capi.HM_DTYPE_INT8 else np.float32)
        return payload.reshape(E, 3, H * I), scale, zp

    def read_router(self, layer: int) -> np.ndarray:
        w = np.empty((self.hidden, self.experts), np.float32)
        _check(load().hm_packed_read_router(self._h, layer, w.ctypes.data, w.size))
        return w

    def load_layer(self, layer: int):
        """(DeviceExpertLayer, router matrix on the device) of one layer."""
        import torch
        from .block import DeviceExpertLayer
        payload, scale, zp = self.read_layer(layer)
        int8 = self.dtype == capi.HM_DTYPE_INT8
        dev = DeviceExpertLayer(payload, scale if int8 else None, zp if int8 else None,
                                self.hidden, self.intermediate)
        return dev, torch.from_numpy(self.read_router(layer)).cuda()


def _align(v: int) -> int:
    return (v + ALIGN - 1) // ALIGN * ALIGN


def write_packed_model(directory, layers, hidden: int, inter: int, top_k: int,
                       renorm: bool = True, softmax: bool = True,
                       model_name: str = "synthetic-moe") -> None:
    """Writes a packed model directory in the reference's format.

    layers: one (experts, router) per layer; experts is a list over expert
    ids of (gate [H x I], up [H x I], down [I x H], quantization), arrays
    row-major INPUT_OUTPUT of int8, float32, float16 or uint16 (the bits of
    BF16), quantization a list of three (scale, zero_point) for INT8 or
    None; router [H x E] FP32."""
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    E = len(layers[0][0])
    tensors, experts_json, routers_json = [], [], []
    records, projections = [], []
    int8 = layers[0][0][0][0].dtype == np.int8
    with open(d / "experts.bin", "wb") as f:
        cursor = 0
        for lid, (experts, _) in enumerate(layers):
            for eid, (g, u, dn, q) in enumerate(experts):
                start = _align(cursor)
                f.write(b"\0" * (start - cursor))
                cursor = start
                blob = b""
                mapping = {"layer_id": lid, "expert_id": eid}
                for p, (role, arr) in enumerate((("gate", g), ("up", u), ("down", dn))):
                    arr = np.ascontiguousarray(arr)
                    data = arr.tobytes()
                    off = start + len(blob)
                    name = f"layers.{lid}.experts.{eid}.{role}"
                    dtype = {np.dtype(np.int8): "INT8", np.dtype(np.float32): "FP32",
                             np.dtype(np.float16): "FP16",
                             np.dtype(np.uint16): "BF16"}[arr.dtype]  # uint16 = bf16 bits
                    t = {"name": name, "source_file": "experts.bin", "offset": off,
                         "size": len(data), "dtype": dtype, "shape": list(arr.shape)}
                    if dtype == "INT8":
                        t["quantization"] = {"scheme": "PER_TENSOR_AFFINE_INT8",
                                             "scale": float(np.float32(q[p][0])),
                                             "zero_point": int(q[p][1])}
                    tensors.append(t)
                    mapping[role] = {"tensor": name, "offset": off, "size": len(data),
                                     "shape": list(arr.shape), "layout": "INPUT_OUTPUT"}
                    projections.append((lid, eid, p, DTYPE_CODE[dtype], 2, 0, off, len(data),
                                        (arr.shape[0], arr.shape[1], 0, 0),
                                        zlib.crc32(data), 0))
                    blob += data
                f.write(blob)
                cursor = start + len(blob)
                records.append((lid, eid, start, len(blob), QUANT_INT8 if int8 else QUANT_FP32,
                                zlib.crc32(blob)))
                experts_json.append(mapping)
        for lid, (_, router) in enumerate(layers):
            r = np.ascontiguousarray(router, np.float32)
            name = f"layers.{lid}.router"
            tensors.append({"name": name, "source_file": "experts.bin", "offset": cursor,
                            "size": r.nbytes, "dtype": "FP32", "shape": list(r.shape)})
            routers_json.append({"layer_id": lid, "tensor": name})
            f.write(r.tobytes())
            cursor += r.nbytes
    write_index(d / "experts.index", records, projections)
    manifest = {
        "schema": "hypermoe.model-manifest.v3", "model_name": model_name,
        "architecture": "QWEN_MOE", "source_architecture": "Qwen3MoeForCausalLM",
        "layer_count": len(layers), "parameter_count": 0, "expert_count": E,
        "hidden_size": hidden, "intermediate_size": inter,
        "capabilities": {"routed_experts": True, "configurable_top_k": True,
                         "normalized_routing": renorm, "gated_expert_mlp": True,
                         "shared_experts": False, "quantized_expert_weights": int8},
        "router": {"expert_count": E, "top_k": top_k,
                   "normalization": "SOFTMAX" if softmax else "NONE",
                   "renormalize_selected": renorm, "layout": "INPUT_OUTPUT",
                   "tensors": routers_json},
        "tensors": tensors, "experts": experts_json, "layers": [],
    }
    with open(d / "manifest.json", "w") as f:
        json.dump(manifest, f, indent=1)
        f.write("\n")


def layers_from_payload(payload: np.ndarray, scale, zp, experts: int, hidden: int, inter: int):
    """Split a synthetic [E x (gate|up|down)] payload (hmoe.synth) into the
    per-expert arrays write_packed_model takes."""
    flat = payload.reshape(-1)
    per = 3 * hidden * inter
    out = []
    for e in range(experts):
        blob = flat[e * per:(e + 1) * per]
        g = blob[:hidden * inter].reshape(hidden, inter)
        u = blob[hidden * inter:2 * hidden * inter].reshape(hidden, inter)
        dn = blob[2 * hidden * inter:].reshape(inter, hidden)
        q = None if scale is None else [(float(scale[e, p]), int(zp[e, p])) for p in range(3)]
        out.append((g, u, dn, q))
    return out


__all__ = ["PackedModel", "StorageError", "crc32", "read_index", "write_index",
           "write_packed_model", "layers_from_payload"]
