"""LLMOE_NUMERICS_FAST against the CPU oracle (the reference's exact restatement).

Fast mode changes two fp32 stages only: the gate_up SiLU (hardware exp / reciprocal / fp16 conversion, the
reference's own __expf / __fdividef / __float2half precision) and the combine (fused into the down GEMM as atomic
adds, summation order free). So:
  - the int32 expert products stay exact: the GPU's A8 of its own Z and the down GEMM + combine are checked against
    the oracle run from that same Z, bit-exact for the A8 codes and within summation-order rounding for the output;
  - Z is within one fp16 rounding step of the exact Z;
  - the layer output is within the contract's max-abs 1e-3 relative tolerance (FP_TOL) of the exact oracle.
"""
import sys

import numpy as np
import pytest

import oracle
from llmoe import Layer, synth

pytestmark = pytest.mark.gpu

FP_TOL = 1e-3        # max |gpu - oracle| <= FP_TOL * max |oracle| (the contract's fp32 tolerance)
ORDER_TOL = 2e-6     # the same slot outputs summed in another order (9 terms, fp32)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def check_fast(G, L, x, lg, pool, out):
    T = x.shape[0]
    S = T * 8 + T
    ref = oracle.Layer(L).forward(x, logits=lg, C=pool)
    topk = G.read("topk", (T, 8), np.int32)
    assert np.array_equal(topk, ref["topk"]), "expert indices differ"
    Z = G.read("Z", (S, 512), np.uint16)
    zg = Z.view(np.float16).astype(np.float64)
    zr = ref["Z"].view(np.float16).astype(np.float64)
    assert np.isfinite(zg).all()
    assert (np.abs(zg - zr) <= np.maximum(np.abs(zg), np.abs(zr)) * 2.0 ** -10 + 6e-8).all(), \
        "fast Z beyond one fp16 rounding step"
    # the rest of the expert stage from the GPU's own Z: A8 bit-exact, output up to the summation order
    rz = oracle.Layer(L).experts_from_z(Z, ref["topk"], ref["topw"])
    assert np.array_equal(G.read("zq", (S, 512), np.int8), rz["zq"]), "A8 of Z differs"
    assert np.array_equal(G.read("zs", (S, 4), np.float32).view(np.uint32), rz["zs"].view(np.uint32))
    e_order = rel_err(out, rz["out"])
    assert e_order <= ORDER_TOL, f"down + combine from the GPU's Z: rel err {e_order}"
    e = rel_err(out, ref["out"])
    assert e <= FP_TOL, f"fast output vs exact oracle: rel err {e}"
    return e


@pytest.mark.parametrize("T,mix,pool,kind", [
    (32, "mixed", 48, None),        # decode: streamed GEMMs, the combine fused into the down GEMM
    (1, "mixed", 256, None),
    (200, "mixed", 48, None),       # several routing blocks: tiled GEMMs
    (512, "mixed", 256, "skewed"),
    (2048, 2, 256, "zipf"),
])
def test_fast_layer(gpu, T, mix, pool, kind):
    import torch
    say(f"[fast] T={T} mix={mix} pool={pool} {kind}")
    L = synth.make_layer(77 + T, mix=mix, shared=True, w8_symmetric=False)
    G = Layer(L["blob"], L["gu_off"], L["d_off"], L["bits"], L["bias"], L["Wr"], pool=pool, has_shared=True,
              max_tokens=max(T, 32))
    G.set_numerics(True)
    x = synth.make_x(5 + T, T)
    lg = None if kind is None else (synth.logits_zipf(T + 3, T) if kind == "zipf" else synth.logits_skewed(T + 3, T))
    out = G.forward(to_dev(x, gpu), None if lg is None else to_dev(lg, gpu))
    torch.cuda.synchronize()
    e = check_fast(G, L, x, lg, pool, out.cpu().numpy())
    say(f"  rel err vs exact oracle {e:.2e}")
    # back to exact: bit-identical to the oracle again
    G.set_numerics(False)
    out = G.forward(to_dev(x, gpu), None if lg is None else to_dev(lg, gpu))
    torch.cuda.synchronize()
    ref = oracle.Layer(L).forward(x, logits=lg, C=pool)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref["out"].view(np.uint32))
    G.close()


@pytest.mark.parametrize("T", [32, 200])
def test_fast_experts_norm(gpu, T):
    """Fast mode with the fused norm epilogue: the combined rows come from the down GEMM's atomic adds."""
    import torch
    say(f"[fast norm] T={T}")
    L = synth.make_layer(91, mix="mixed", shared=True)
    G = Layer(L["blob"], L["gu_off"], L["d_off"], L["bits"], L["bias"], L["Wr"], pool=48, has_shared=True,
              max_tokens=256)
    G.set_numerics(True)
    x = synth.make_x(900 + T, T)
    signs = np.where(np.random.default_rng(T).random(2048) < 0.5, -1.0, 1.0).astype(np.float32)
    h0 = (np.random.default_rng(T + 1).standard_normal((T, 2048)) * 2).astype(np.float32)
    xq, xs, xsum = oracle.quant_a8(x)
    dx = [to_dev(a, gpu) for a in (xq, xs, xsum)]
    G.route(T, x=to_dev(x, gpu))
    h = to_dev(h0, gpu)
    q, s, sm = G.experts_norm(*dx, to_dev(signs, gpu), 1e-6, h)
    torch.cuda.synchronize()
    r = oracle.Layer(L).forward(x, C=48)
    hn, rq, rs, rsm = oracle.combine_norm(r["Y"], r["tok_slots"], 9, signs, 1e-6, h0)
    assert rel_err(h.cpu().numpy() - h0, hn - h0) <= FP_TOL, "residual update beyond tolerance"
    # the next layer's A8 codes of a tolerance-close input: nearly all equal, none off by more than one
    dq = np.abs(q.cpu().numpy().astype(int) - rq.astype(int))
    assert dq.max() <= 1 and (dq > 0).mean() < 0.01
    G.close()
