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
