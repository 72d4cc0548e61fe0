"""Python host mirror of the MoE-block entry over the C ABI.

`DeviceExpertLayer` uploads one layer of experts (the reference payload
layout, ExpertPacker.cpp:228-230) and packs it on the device once
(hm_pack_layer).  `MoEBlock.execute_batch` mirrors
MoERuntime::executeBatch (src/core/runtime/MoERuntime.cpp:58-349): it returns
the routing (ids/scores per token), the expert groups (ExpertBatch: expert id,
token indices, routing weights), the per-group expert outputs and the
combined output, like BatchLayerExecutionResult (MoERuntime.hpp:33-39).
Device memory and the stream come from torch; all compute is the HIP
library.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import capi

ROUTE_SOFTMAX = capi.HM_ROUTE_SOFTMAX
ROUTE_RENORM = capi.HM_ROUTE_RENORM


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("the MoE block needs a GPU (HIP); there is no CPU fallback")
    return torch


class DeviceExpertLayer:
    """All experts of one layer, resident in HBM in the kernels' layout."""

    def __init__(self, payload: np.ndarray, scale: np.ndarray | None, zp: np.ndarray | None,
                 hidden: int, inter: int, stream=None):
        torch = _torch()
        self.experts = payload.shape[0]
        self.hidden, self.inter = hidden, inter
        self.int8 = payload.dtype == np.int8
        if payload.size != self.experts * 3 * hidden * inter:
            raise ValueError("payload does not match [E, 3, H*I]")
        dtype = capi.HM_DTYPE_INT8 if self.int8 else capi.HM_DTYPE_FP32
        self.dtype = dtype
        src = torch.from_numpy(np.ascontiguousarray(payload)).to("cuda")
        nbytes = capi.load().hm_packed_layer_bytes(self.experts, hidden, inter, dtype)
        if nbytes == 0:
            raise ValueError("invalid expert layer shape")
        self.packed = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        capi.call("hm_pack_layer", src.data_ptr(), self.experts, hidden, inter, dtype,
                  self.packed.data_ptr(), s)
        torch.cuda.synchronize()
        del src
        if self.int8:
            self.scale = torch.from_numpy(np.ascontiguousarray(scale, np.float32)).to("cuda")
            self.zp = torch.from_numpy(np.ascontiguousarray(zp, np.int32)).to("cuda")
        else:
            self.scale = self.zp = None
        self.desc = capi.HmLayer(self.experts, hidden, inter, dtype, self.packed.data_ptr(),
                                 self.scale.data_ptr() if self.int8 else None,
                                 self.zp.data_ptr() if self.int8 else None)


@dataclass
class ExpertBatch:
    """ExpertBatch (src/experts/ExpertBatch.hpp:10-18)."""
    expert_id: int
    token_indices: np.ndarray
    routing_weights: np.ndarray


@dataclass
class BlockResult:
    ids: np.ndarray             # [T, k] rank order (RouterDecision.selectedExpertIds)
    scores: np.ndarray          # [T, k]           (RouterDecision.routingScores)
    counts: np.ndarray          # [E]
    offsets: np.ndarray         # [E+1]
    perm_tokens: np.ndarray     # [T*k] group order
    perm_weights: np.ndarray    # [T*k]
    status: int
    output: object              # torch [T, H] on the device
    expert_out: object = None   # torch [T*k, H] grouped order
    batches: list = field(default_factory=list)


class MoEBlock:
    def __init__(self, layer: DeviceExpertLayer, top_k: int, softmax: bool = True,
                 renorm: bool = True, limbs_x: int = 2, limbs_z: int = 3):
        self.layer, self.top_k = layer, top_k
        self.flags = (ROUTE_SOFTMAX if softmax else 0) | (ROUTE_RENORM if renorm else 0)
        self.limbs_x, self.limbs_z = limbs_x, limbs_z
        self._ws = None
        self._ws_tokens = -1
        self._io_bufs = None

    def _buffers(self, tokens: int, exec_flags: int = 0):
        torch = _torch()
        nbytes = capi.load().hm_moe_block_workspace_bytes(
            C.byref(self.layer.desc), tokens, self.top_k, self.limbs_x, self.limbs_z, exec_flags)
        if nbytes == 0:
            raise ValueError("invalid block configuration")
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        if self._ws_tokens != tokens:
            P, E, H = tokens * self.top_k, self.layer.experts, self.layer.hidden
            self._io_bufs = dict(
                out=torch.empty((tokens, H), dtype=torch.float32, device="cuda"),
                ids=torch.empty((tokens, self.top_k), dtype=torch.int32, device="cuda"),
                scores=torch.empty((tokens, self.top_k), dtype=torch.float32, device="cuda"),
                counts=torch.empty(E, dtype=torch.int32, device="cuda"),
                offsets=torch.empty(E + 1, dtype=torch.int32, device="cuda"),
                perm_tokens=torch.empty(P, dtype=torch.int32, device="cuda"),
                perm_weights=torch.empty(P, dtype=torch.float32, device="cuda"),
                expert_out=torch.empty((P, H), dtype=torch.float32, device="cuda"),
                status=torch.zeros(1, dtype=torch.int32, device="cuda"),
            )
            self._ws_tokens = tokens
        return self._ws, self._io_bufs

    def launch(self, hidden, router_w, residual=None, exec_flags: int = 0, stream=None,
               events=None):
        """Asynchronous launch on `stream` (default: torch's current stream).
        `events`: optional HM_BLOCK_EVENTS hipEvent_t handles (ints) recorded
        at the stage boundaries."""
        torch = _torch()
        tokens = hidden.shape[0]
        ws, b = self._buffers(tokens, exec_flags)
        # b["status"] starts at zero and kernels only OR bits into it;
        # execute_batch clears it after reporting a failure
        io = capi.HmBlockIO(b["out"].data_ptr(), b["ids"].data_ptr(), b["scores"].data_ptr(),
                            b["counts"].data_ptr(), b["offsets"].data_ptr(),
                            b["perm_tokens"].data_ptr(), b["perm_weights"].data_ptr(),
                            b["expert_out"].data_ptr(), b["status"].data_ptr(),
                            residual.data_ptr() if residual is not None else None)
        if events is not None:
            arr = (C.c_void_p * capi.HM_BLOCK_EVENTS)(*events)
            io.events = C.cast(arr, C.POINTER(C.c_void_p))
            self._event_arr = arr  # keep alive through the call
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        capi.call("hm_moe_block_forward", C.byref(self.layer.desc), hidden.data_ptr(),
                  router_w.data_ptr(), tokens, self.top_k, self.flags | exec_flags,
                  self.limbs_x, self.limbs_z, C.byref(io), ws.data_ptr(), ws.numel(), s)
        return b

    def execute_batch(self, hidden, router_w, residual=None, exec_flags: int = 0) -> BlockResult:
        torch = _torch()
        b = self.launch(hidden, router_w, residual, exec_flags)
        torch.cuda.synchronize()
        status = int(b["status"].cpu().item())
        if status:
            b["status"].zero_()
            raise RuntimeError(f"router failed on the device (status bits {status:#x})")
        res = BlockResult(
            ids=b["ids"].cpu().numpy().view(np.uint32), scores=b["scores"].cpu().numpy(),
            counts=b["counts"].cpu().numpy(), offsets=b["offsets"].cpu().numpy(),
            perm_tokens=b["perm_tokens"].cpu().numpy(),
            perm_weights=b["perm_weights"].cpu().numpy(), status=status,
            # callee-allocated results (MoERuntime.cpp:134): the next call
            # reuses the block's buffers
            output=b["out"].clone(), expert_out=b["expert_out"].clone())
        for e in range(self.layer.experts):
            lo, hi = res.offsets[e], res.offsets[e + 1]
            if hi > lo:
                res.batches.append(ExpertBatch(e, res.perm_tokens[lo:hi].copy(),
                                               res.perm_weights[lo:hi].copy()))
        return res
