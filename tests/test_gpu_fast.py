"""LLMOE_NUMERICS_FAST against the CPU oracle (the reference's exact restatement).

Fast mode changes two fp32 stages: the gate_up SiLU (hardware exp / reciprocal / fp16 conversion, the reference's
own __expf / __fdividef / __float2half precision), and, with several routing blocks (T > 32), the down GEMM's slot
outputs Y, stored as fp16 (round to nearest even) for the combine. So:
  - Z is within one fp16 rounding step of the exact Z;
  - everything after gate_up is exact given that Z: the GPU's A8 of its own Z, the fp16 slot outputs Y (its int32
    products and epilogue, then the rounding) and the combine are bit-identical to the oracle run from the same Z
    (experts_from_z, y_half=True when T > 32);
  - the layer output is within the contract's max-abs 1e-3 relative tolerance (FP_TOL) of the exact oracle.
"""
import sys

import numpy as np
import pytest

import oracle
from llmoe import Layer, synth

pytestmark = pytest.mark.gpu

FP_TOL = 1e-3        # max |gpu - oracle| <= FP_TOL * max |oracle| (the contract's fp32 tolerance)


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


def read_y(G, S, T):
    """The fast-mode slot outputs as fp32 values: fp16 [S, 2048] in the Y buffer when T > 32 (several routing
    blocks), fp32 otherwise."""
    if T > 32:
        return G.read("Y", (S, 2048), np.uint16).view(np.float16).astype(np.float32)
    return G.read("Y", (S, 2048), np.float32)


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
    # the rest of the expert stage from the GPU's own Z: bit-exact
    rz = oracle.Layer(L).experts_from_z(Z, ref["topk"], ref["topw"], y_half=T > 32)
    assert np.array_equal(G.read("zq", (S, 512), np.int8), rz["zq"]), "A8 of Z differs"
    assert np.array_equal(G.read("zs", (S, 4), np.float32).view(np.uint32), rz["zs"].view(np.uint32))
    yh = read_y(G, S, T)
    assert np.array_equal(yh.view(np.uint32), rz["Y"].view(np.uint32)), "down GEMM from the GPU's Z differs"
    assert np.array_equal(out.view(np.uint32), rz["out"].view(np.uint32)), "combine differs"
    e = rel_err(out, ref["out"])
    assert e <= FP_TOL, f"fast output vs exact oracle: rel err {e}"
    return e


@pytest.mark.parametrize("T,mix,pool,kind", [
    (32, "mixed", 48, None),        # decode: streamed GEMMs
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
    """Fast mode with the fused norm epilogue, against the oracle's combine + norm of the GPU's own slot outputs."""
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
    S = 9 * T
    Y = read_y(G, S, T)
    ts = G.read("tok_slots", (T, 9), np.int32)
    hn, rq, rs, rsm = oracle.combine_norm(Y, ts, 9, signs, 1e-6, h0)
    assert np.array_equal(h.cpu().numpy().view(np.uint32), hn.view(np.uint32)), "residual not bit-exact"
    assert np.array_equal(q.cpu().numpy(), rq)
    r = oracle.Layer(L).forward(x, C=48)
    hr, _, _, _ = oracle.combine_norm(r["Y"], r["tok_slots"], 9, signs, 1e-6, h0)
    assert rel_err(h.cpu().numpy() - h0, hr - h0) <= FP_TOL, "residual update beyond tolerance vs exact"
    G.close()
