"""llmoe_experts_scratch (the expert stage with its intermediates in the library's static per-GPU array, no
allocation) against llmoe_experts on the same routing, through the C ABI: bit-exact, on two calls in a row, the
second with fewer tokens (the array keeps the first call's contents), plus the size limit."""
import sys

import numpy as np
import pytest

import llmoe
import oracle
from llmoe import Layer, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_experts_scratch_matches_experts(gpu):
    import torch
    L = synth.make_layer(11, mix="mixed", shared=True)
    G = Layer(L["blob"], L["gu_off"], L["d_off"], L["bits"], L["bias"], L["Wr"], pool=48, has_shared=True,
              max_tokens=128)
    for T in (llmoe.SCRATCH_MAX_TOKENS, 20):
        say(f"[no_alloc] T={T}")
        x = synth.make_x(300 + T, T)
        xq, xs, xsum = (torch.from_numpy(a).to(gpu) for a in oracle.quant_a8(x))
        G.route(T, x=torch.from_numpy(x).to(gpu))
        a = G.experts(xq, xs, xsum)
        b = G.experts_scratch(xq, xs, xsum)
        torch.cuda.synchronize()
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"T={T}: scratch path differs"
        r = oracle.Layer(L).forward(x, C=48)
        assert np.array_equal(b.view(np.uint32), r["out"].view(np.uint32)), f"T={T}: differs from the oracle"
    # beyond the static array: a clear error, nothing launched
    T = llmoe.SCRATCH_MAX_TOKENS + 1
    x = synth.make_x(7, T)
    xq, xs, xsum = (torch.from_numpy(a).to(gpu) for a in oracle.quant_a8(x))
    G.route(T, x=torch.from_numpy(x).to(gpu))
    with pytest.raises(RuntimeError, match="static scratch"):
        G.experts_scratch(xq, xs, xsum)
    torch.cuda.synchronize()
    G.close()


def test_experts_scratch_graph_replays(gpu):
    """llmoe_experts_scratch captured in a HIP graph together with its routing: every replay, after eager calls that
    overwrite the static array with another input's intermediates, reproduces the eager output bit for bit (the
    array's device address is looked up when the layer is created, not during capture)."""
    import torch
    say("[no_alloc] graph capture T=32")
    L = synth.make_layer(12, mix="mixed", shared=True)
    G = Layer(L["blob"], L["gu_off"], L["d_off"], L["bits"], L["bias"], L["Wr"], pool=48, has_shared=True,
              max_tokens=64)
    T = 32
    x_np, x2_np = synth.make_x(400, T), synth.make_x(401, T)
    x, x2 = torch.from_numpy(x_np).to(gpu), torch.from_numpy(x2_np).to(gpu)
    q1 = [torch.from_numpy(a).to(gpu) for a in oracle.quant_a8(x_np)]
    q2 = [torch.from_numpy(a).to(gpu) for a in oracle.quant_a8(x2_np)]
    out = torch.empty((T, 2048), dtype=torch.float32, device=gpu)
    G.route(T, x=x)
    G.experts_scratch(*q1, out=out)
    torch.cuda.synchronize()
    ref = out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        G.route(T, x=x)
        G.experts_scratch(*q1, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        G.route(T, x=x)
        G.experts_scratch(*q1, out=out)
    for i in range(4):
        out.zero_()
        G.route(T, x=x2)                      # eager: other routing and other intermediates in the array
        other = G.experts_scratch(*q2)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"replay {i}: output differs"
        assert not torch.equal(other, ref)
    del g
    r = oracle.Layer(L).forward(x_np, C=48)
    assert np.array_equal(ref.cpu().numpy().view(np.uint32), r["out"].view(np.uint32)), "differs from the oracle"
    G.close()
