"""A stack of MoE blocks with RMSNorm and residual (the C5 configuration).

Each layer is TransformerBlock::execute with attention omitted
(src/transformer/runtime/TransformerBlock.cpp:88-104):
    h' = h + MoE(RMSNorm(h))
with RMSNorm as RMSNorm::execute (src/transformer/norm/RMSNorm.cpp:65-77)
and the MoE block as MoERuntime::executeBatch.  Everything runs through the
C ABI on one stream: one hm_moe_layer_forward per layer (the RMSNorm
folded into the router's first kernel for decode batches, launched ahead of
the block otherwise; the residual folded into the combine).  The layers share one block workspace and
one device status word; the residual stream ping-pongs between two buffers
so that a layer's output never aliases its residual input.  A decode step
issues no allocation and no synchronisation, so it can be captured in a HIP
graph and replayed.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import capi
from .block import DeviceExpertLayer


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("the MoE stack needs a GPU (HIP); there is no CPU fallback")
    return torch


class MoEStack:
    def __init__(self, layers: list[DeviceExpertLayer], router_w: list, top_k: int,
                 eps: float = 1e-6, limbs_x: int = 2, limbs_z: int = 3,
                 flags: int = capi.HM_ROUTE_SOFTMAX | capi.HM_ROUTE_RENORM):
        torch = _torch()
        if not layers or len(layers) != len(router_w):
            raise ValueError("one router matrix per layer")
        h0 = layers[0].hidden
        if any(l.hidden != h0 for l in layers):
            raise ValueError("all layers share the hidden size")
        self.layers, self.router_w = layers, router_w
        self.top_k, self.eps, self.flags = top_k, eps, flags
        self.limbs_x, self.limbs_z = limbs_x, limbs_z
        self.hidden = h0
        self.gamma = torch.ones(h0, dtype=torch.float32, device="cuda")
        self.status = torch.zeros(1, dtype=torch.int32, device="cuda")
        self._tokens = -1

    def _buffers(self, tokens: int):
        torch = _torch()
        if tokens == self._tokens:
            return
        need = 0
        for l in self.layers:
            need = max(need, capi.load().hm_moe_block_workspace_bytes(
                C.byref(l.desc), tokens, self.top_k, self.limbs_x, self.limbs_z, 0))
        if need == 0:
            raise ValueError("invalid stack configuration")
        self.ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        self.norm = torch.empty((tokens, self.hidden), dtype=torch.float32, device="cuda")
        self.ping = [torch.empty((tokens, self.hidden), dtype=torch.float32, device="cuda")
                     for _ in range(2)]
        self._tokens = tokens

    def launch(self, h, events=None, stream=None):
        """Run every layer on h [tokens x hidden] (device, float32) and return
        the output buffer (one of two internal buffers, valid until the next
        launch).  `events`: optional list of len(layers)+1 torch events
        recorded before layer 0 and after each layer."""
        torch = _torch()
        tokens = h.shape[0]
        self._buffers(tokens)
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        lib = capi.load()
        cur = h
        if events is not None:
            events[0].record()
        for i, (layer, w) in enumerate(zip(self.layers, self.router_w)):
            out = self.ping[i & 1]
            io = capi.HmBlockIO(out.data_ptr(), None, None, None, None, None, None, None,
                                self.status.data_ptr(), None)
            # RMSNorm, the block and the residual in one call (the norm runs
            # inside the router's first kernel for decode batches)
            capi.call("hm_moe_layer_forward", C.byref(layer.desc), cur.data_ptr(),
                      self.gamma.data_ptr(), self.eps, self.norm.data_ptr(), w.data_ptr(),
                      tokens, self.top_k, self.flags, self.limbs_x, self.limbs_z, C.byref(io),
                      self.ws.data_ptr(), self.ws.numel(), s)
            cur = out
            if events is not None:
                events[i + 1].record()
        del lib
        return cur

    def check_status(self):
        """Raise if a kernel of any layer reported a routing failure since the
        last check (the reference throws at CpuRouterBackend.cpp:47/57/83)."""
        torch = _torch()
        torch.cuda.synchronize()
        st = int(self.status.cpu().item())
        if st:
            self.status.zero_()
            raise RuntimeError(f"router failed on the device (status bits {st:#x})")


def build_stack(cfg, seed: int | None = None, layers: int | None = None, limbs_x: int = 2,
                limbs_z: int = 3, log=None) -> MoEStack:
    """The seeded INT8 stack of a configuration (synth.CONFIGS): per layer the
    packed experts and the router matrix, generated on the host by the
    synthetic generator and kept resident on the device."""
    torch = _torch()
    from . import synth
    seed = cfg.seed if seed is None else seed
    n = cfg.layers if layers is None else layers
    dev_layers, routers = [], []
    for l in range(n):
        payload, scale, zp = synth.expert_layer(seed, l, cfg.experts, cfg.hidden, cfg.inter,
                                                cfg.int8)
        dev_layers.append(DeviceExpertLayer(payload, scale, zp, cfg.hidden, cfg.inter))
        del payload
        w = synth.router_weights(seed, l, cfg.hidden, cfg.experts)
        routers.append(torch.from_numpy(np.ascontiguousarray(w)).to("cuda"))
        if log is not None:
            log(l)
    return MoEStack(dev_layers, routers, cfg.top_k, limbs_x=limbs_x, limbs_z=limbs_z)
