"""hm_moe_block_forward_noalloc: the MoE block with its workspace in the
library's own device array (for callers that cannot allocate).  Called
through the C ABI and checked bit for bit against hm_moe_block_forward on
the same inputs, on two calls in a row (the second with a smaller batch, so
it runs over what the first left in the array), for the INT8 prefill path,
the decode path and FP32 experts; a batch whose workspace exceeds the array
is refused before anything is launched."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact
from hmoe import capi, synth
from hmoe.block import DeviceExpertLayer, MoEBlock

pytestmark = pytest.mark.gpu


def _inputs(seed, T, H, E, I, int8):
    payload, scale, zp = synth.expert_layer(seed, 0, E, H, I, int8)
    h = O.rmsnorm(synth.raw_hidden(seed, T, H), np.ones(H, np.float32))
    w = synth.router_weights(seed, 0, H, E)
    return payload, scale, zp, h, w


def _noalloc(block, h, w, exec_flags=0):
    """One call of the no-allocation entry with fresh output buffers."""
    import torch
    T, H, k, E = h.shape[0], block.layer.hidden, block.top_k, block.layer.experts
    P = T * k
    out = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
    ids = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
    scores = torch.empty((T, k), dtype=torch.float32, device="cuda")
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    ptok = torch.empty(P, dtype=torch.int32, device="cuda")
    pw = torch.empty(P, dtype=torch.float32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    io = capi.HmBlockIO(out.data_ptr(), ids.data_ptr(), scores.data_ptr(), counts.data_ptr(),
                        offsets.data_ptr(), ptok.data_ptr(), pw.data_ptr(), None,
                        status.data_ptr(), None)
    stream = torch.cuda.current_stream().cuda_stream
    capi.call("hm_moe_block_forward_noalloc", C.byref(block.layer.desc), h.data_ptr(),
              w.data_ptr(), T, k, block.flags | exec_flags, block.limbs_x, block.limbs_z,
              C.byref(io), stream)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    return (out.cpu().numpy(), ids.cpu().numpy().view(np.uint32), scores.cpu().numpy(),
            ptok.cpu().numpy())


@pytest.mark.parametrize("int8,T1,T2", [(True, 200, 37), (True, 16, 3), (False, 40, 9)])
def test_noalloc_matches_block_forward(dev, int8, T1, T2):
    import torch
    H, E, I, k = 2048, 64, 768, 8
    print(f"[gpu] noalloc int8={int8} T={T1} then T={T2}", flush=True)
    payload, scale, zp, h, w = _inputs(5 + T1, T1, H, E, I, int8)
    layer = DeviceExpertLayer(payload, scale if int8 else None, zp if int8 else None, H, I)
    block = MoEBlock(layer, k)
    dw = torch.from_numpy(w).cuda()
    for T in (T1, T2):
        need = capi.load().hm_moe_block_workspace_bytes(C.byref(layer.desc), T, k, 2, 2, 0)
        assert 0 < need <= capi.HM_NOALLOC_WORKSPACE_BYTES
        dh = torch.from_numpy(np.ascontiguousarray(h[:T])).cuda()
        ref = block.execute_batch(dh, dw)
        out, ids, scores, ptok = _noalloc(block, dh, dw)
        assert_bitexact(ids, ref.ids, f"T={T} ids")
        assert_bitexact(scores, ref.scores, f"T={T} scores")
        assert_bitexact(ptok, ref.perm_tokens, f"T={T} permutation")
        assert_bitexact(out, ref.output.cpu().numpy(), f"T={T} output")


def test_noalloc_refuses_oversized_batch(dev):
    """A batch whose workspace exceeds the array returns HM_ERR_UNSUPPORTED
    and launches nothing (the output buffer keeps its contents)."""
    import torch
    H, E, I, k, T = 2048, 128, 768, 8, 4096
    desc = capi.HmLayer(E, H, I, capi.HM_DTYPE_INT8, 1, 1, 1)  # never dereferenced
    need = capi.load().hm_moe_block_workspace_bytes(C.byref(desc), T, k, 2, 2, 0)
    assert need > capi.HM_NOALLOC_WORKSPACE_BYTES
    out = torch.full((4,), 7.0, dtype=torch.float32, device="cuda")
    io = capi.HmBlockIO(out.data_ptr(), None, None, None, None, None, None, None, None, None)
    rc = capi.status("hm_moe_block_forward_noalloc", C.byref(desc), 1, 1, T, k,
                     capi.HM_ROUTE_SOFTMAX | capi.HM_ROUTE_RENORM, 2, 2, C.byref(io), None)
    assert rc == capi.HM_ERR_UNSUPPORTED
    torch.cuda.synchronize()
    assert out.cpu().tolist() == [7.0] * 4
