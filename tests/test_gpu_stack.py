"""GPU parity for the C5 stack (A12 + A1 + the MoE block per layer):
h' = h + MoE(RMSNorm(h)) per layer (TransformerBlock.cpp:88-104, attention
omitted), checked layer by layer against the CPU oracle fed the device's
own layer input, and the captured decode step replayed against eager."""
from __future__ import annotations

import numpy as np
import pytest

import hm_oracle as O
from conftest import assert_bitexact, normwise
from hmoe import synth
from hmoe.block import MoEBlock
from hmoe.stack import MoEStack, build_stack

pytestmark = pytest.mark.gpu

SMALL = synth.Config("stack-small", tokens=40, hidden=512, experts=16, top_k=4, inter=256,
                     layers=3, seed=77)


@pytest.fixture(scope="module")
def small_stack():
    import torch
    stack = build_stack(SMALL)
    host = []
    for l in range(SMALL.layers):
        payload, scale, zp = synth.expert_layer(SMALL.seed, l, SMALL.experts, SMALL.hidden,
                                                SMALL.inter, True)
        host.append((payload, scale, zp, synth.router_weights(SMALL.seed, l, SMALL.hidden,
                                                              SMALL.experts)))
    yield stack, host
    del stack
    torch.cuda.synchronize()


@pytest.mark.parametrize("T", [40, 1])
def test_stack_layers_vs_oracle(small_stack, T):
    """Each layer's output equals h + MoE_ref(RMSNorm(h)) for its device input
    h: routing bit-exact, the MoE part within 1e-4 normwise; the full stack
    launch gives the same bits as the layers launched one at a time."""
    import torch
    stack, host = small_stack
    print(f"[gpu] stack T={T} layers={SMALL.layers}", flush=True)
    rng = np.random.default_rng(T)
    h = rng.standard_normal((T, SMALL.hidden)).astype(np.float32)
    cur = torch.from_numpy(h).cuda()
    gamma = np.ones(SMALL.hidden, np.float32)
    for l in range(SMALL.layers):
        one = MoEStack([stack.layers[l]], [stack.router_w[l]], SMALL.top_k)
        out = one.launch(cur).clone()
        one.check_status()
        h_in = cur.cpu().numpy()
        payload, scale, zp, w = host[l]
        hn = O.rmsnorm(h_in, gamma)
        moe_ref, ids, _ = O.moe_block(payload, scale, zp, hn, w, SMALL.top_k, SMALL.inter)
        res = MoEBlock(stack.layers[l], SMALL.top_k).execute_batch(
            torch.from_numpy(hn).cuda(), stack.router_w[l])
        assert_bitexact(res.ids, ids, f"layer {l} routing")
        got = out.cpu().numpy()
        moe_dev = got.astype(np.float64) - h_in.astype(np.float64)
        assert normwise(moe_dev, moe_ref) < 1e-4, f"layer {l}"
        ref = (h_in + moe_ref).astype(np.float32)
        assert np.max(np.abs(got - ref)) <= 1e-4 * max(1.0, float(np.max(np.abs(ref))))
        cur = out
    full = stack.launch(torch.from_numpy(h).cuda()).clone()
    stack.check_status()
    assert_bitexact(full.cpu().numpy(), cur.cpu().numpy(), "stack launch vs layer by layer")


def test_stack_decode_graph_replay(small_stack):
    """A decode step (one token through every layer) captured in a HIP graph
    and replayed equals the eager step, on every replay."""
    import torch
    stack, _ = small_stack
    rng = np.random.default_rng(3)
    h = torch.from_numpy(rng.standard_normal((1, SMALL.hidden)).astype(np.float32)).cuda()
    static_in = h.clone()
    eager = stack.launch(static_in).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        stack.launch(static_in)  # warm the buffers outside the capture
        with torch.cuda.graph(g, stream=s):
            out = stack.launch(static_in)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert_bitexact(out.cpu().numpy(), eager.cpu().numpy(), f"replay {rep}")
        _ = stack.launch(static_in)  # eager work between replays
        torch.cuda.synchronize()
    stack.check_status()
