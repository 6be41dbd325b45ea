"""CPU tests of the oracle (the checker of the GPU path): pinned against the golden fixtures written by the
reference's own Python (tests/golden/make_golden.py), against closed forms, brute force and numpy."""
from __future__ import annotations

import math
import struct
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from llmoe import synth

GOLD = Path(__file__).resolve().parent / "golden"
import sys
sys.path.insert(0, str(GOLD))
import gen  # noqa: E402
sys.path.insert(0, str(Path(__file__).resolve().parent))
from stages_f64 import check_stages_f64  # noqa: E402


def fixture(name):
    return np.load(GOLD / name, allow_pickle=False)


# ---- packlib "i8" format (quant/packlib.py:140-234) -------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_pack_i8_matches_reference_bytes(bits):
    f = fixture("packlib_i8.npz")
    c, s, z = gen.pack_case(bits)
    assert str(f[f"digest{bits}"]) == gen.digest(c, s, z), "generator drifted from the fixture"
    blob = O.pack_i8(c, s, z, bits)
    assert blob.size == O.matrix_bytes(*gen.PACK_SHAPE, bits)
    np.testing.assert_array_equal(blob, f[f"blob{bits}"])
    c2, s2, z2 = O.unpack_i8(f[f"blob{bits}"], *gen.PACK_SHAPE, bits)
    np.testing.assert_array_equal(c2, c)
    np.testing.assert_array_equal(s2.view(np.uint16), s.view(np.uint16))
    np.testing.assert_array_equal(z2, z)


def test_matrix_bytes_closed_form():
    # quant/packlib.py:33-41: (R/16)(K/128)(tile weight bytes + 48)
    for bits, tw in ((2, 512), (3, 768), (4, 1024), (8, 2048)):
        assert O.matrix_bytes(1024, 2048, bits) == 64 * 16 * (tw + 48)
        assert synth.matrix_bytes(1024, 2048, bits) == O.matrix_bytes(1024, 2048, bits)
    # per-expert packed bytes (gate_up 1024 tiles + down 512 tiles)
    assert [synth.expert_bytes(b) for b in (2, 3, 4, 8)] == [860160, 1253376, 1646592, 3219456]


def test_gu_row_perm_matches_reference():
    np.testing.assert_array_equal(O.gu_row_perm(512), fixture("packlib_i8.npz")["gu_row_perm512"])


def test_pack_single_code_position():
    # One non-zero code lands in exactly one byte / bit field; a dropped or transposed index moves it.
    for bits in (2, 3, 4, 8):
        for (r, k) in ((0, 0), (9, 37), (15, 127), (3, 64), (12, 100)):
            c = np.zeros((16, 128), np.uint8)
            c[r, k] = (1 << bits) - 1
            blob = O.pack_i8(c, np.zeros((16, 1), np.float16), np.zeros((16, 1), np.uint8), bits)
            w = blob[:O.matrix_bytes(16, 128, bits) - 48]
            assert 1 <= int(np.unpackbits(w).sum()) == bits
            c2, _, _ = O.unpack_i8(blob, 16, 128, bits)
            np.testing.assert_array_equal(c2, c)


# ---- A8 (engine/ops.cu:42-66, engine/tests/gen_moe_case.py:24-29) ------------------------------------------
def test_quant_a8_matches_reference():
    f = fixture("a8_fwht.npz")
    rows = gen.a8_rows()
    assert str(f["a8_in_digest"]) == gen.digest(rows)
    q, s, sm = O.quant_a8(rows)
    deq = (q.reshape(8, 4, 128).astype(np.float32) * s[:, :, None]).reshape(8, 512)
    np.testing.assert_array_equal(deq, f["a8_out"])
    np.testing.assert_array_equal(sm, q.reshape(8, 4, 128).astype(np.int32).sum(-1))
    assert np.abs(q.astype(np.int32)).max() <= 127


def test_quant_a8_edge_cases():
    rows = gen.a8_rows()
    q, s, _ = O.quant_a8(rows)
    assert (q[0] == 0).all() and (s[0] == np.float32(1e-30)).all()        # zero rows: floor scale
    # row 1, group 1: values 0.5 + j/2 and a -127 entry, so s = 1 and every even j is an exact .5 tie
    assert s[1, 1] == np.float32(1.0)
    v = rows[1, 128:256]
    np.testing.assert_array_equal(q[1, 128:256], np.rint(v).astype(np.int8))
    assert q[1, 128] == 0 and q[1, 130] == 2 and q[1, 132] == 2           # 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    assert q[5].tolist() == [127, -127] * 256


# ---- FWHT-512 (engine/moe_i8.cu:444-502) -------------------------------------------------------------------
def test_fwht512_matches_reference_hadamard():
    f = fixture("a8_fwht.npz")
    v = gen.fwht_rows()
    assert str(f["fwht_in_digest"]) == gen.digest(v)
    out = np.stack([O.fwht512(r) for r in v])
    np.testing.assert_allclose(out, f["fwht_out"], rtol=0, atol=2e-5 * np.abs(f["fwht_out"]).max())


def test_fwht512_closed_forms():
    i = np.arange(512)
    for k in (0, 1, 77, 511):
        e = np.zeros(512, np.float32)
        e[k] = 1.0
        row = np.array([(-1) ** bin(k & j).count("1") for j in i], np.float64) / math.sqrt(512)
        np.testing.assert_allclose(O.fwht512(e), row, atol=1e-7)
    v = gen.normal(50, (512,)).astype(np.float32)
    np.testing.assert_allclose(O.fwht512(O.fwht512(v)), v, atol=1e-5)      # H H = I after the 1/sqrt(n)


def test_fwht_a8_reciprocal_quantiser():
    Z = gen.normal(51, (6, 512)).astype(np.float16)
    q, s, sm = O.fwht_a8(Z.view(np.uint16))
    for n in range(6):
        v = O.fwht512(Z[n].astype(np.float32))
        for g in range(4):
            vg = v[128 * g:128 * g + 128]
            sc = max(np.float32(np.abs(vg).max()) / np.float32(127), np.float32(1e-30))
            assert s[n, g] == np.float32(sc)
            inv = np.float32(1) / np.float32(sc)
            np.testing.assert_array_equal(q[n, 128 * g:128 * g + 128], np.clip(np.rint(vg * inv), -127, 127))
            assert sm[n, g] == int(q[n, 128 * g:128 * g + 128].astype(np.int32).sum())


# ---- routing (engine/ops.cu:256-327, quant/s03_teacher_pass.py:132-146) -------------------------------------
@pytest.mark.parametrize("C", [48, 256])
def test_route_matches_reference(C):
    f = fixture("route.npz")
    logits, bias = gen.route_case()
    assert str(f["digest"]) == gen.digest(logits, bias)
    topk, topw = O.route(logits, bias, K=8, C=C, block=32, rscale=2.5)
    np.testing.assert_array_equal(topk, f[f"topk{C}"])
    np.testing.assert_allclose(topw, f[f"topw{C}"], rtol=1e-6, atol=0)


def brute_route(logits, bias, K, C, block, rscale):
    sig = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    s = sig + bias
    T, E = s.shape
    topk = np.zeros((T, K), np.int32)
    for b0 in range(0, T, block):
        bm = s[b0:b0 + block].max(0)
        pool = sorted(range(E), key=lambda e: (-bm[e], e))[:C]
        for t in range(b0, min(T, b0 + block)):
            topk[t] = sorted(pool, key=lambda e: (-s[t, e], e))[:K]
    w = np.take_along_axis(sig, topk, 1)
    return topk, w / (w.sum(1, keepdims=True) + 1e-20) * rscale


def test_route_ties_lower_index_first():
    T, E = 40, 64
    lg = np.zeros((T, E), np.float32)
    lg[:, ::3] = 1.0                        # many exact ties in the score and in the block maxima
    lg[5, 60] = 2.0
    bias = np.zeros(E, np.float32)
    for C in (8, 16, 64):
        topk, topw = O.route(lg, bias, K=8, C=C, block=32, rscale=2.5)
        bt, bw = brute_route(lg, bias, 8, C, 32, 2.5)
        np.testing.assert_array_equal(topk, bt)
        np.testing.assert_allclose(topw, bw, rtol=1e-6)


def test_route_random_vs_brute_force():
    lg = (gen.normal(60, (70, 256)) * 2).astype(np.float32)
    bias = gen.uniform(61, (256,), -0.1, 0.1).astype(np.float32)
    for C in (48, 256):
        topk, topw = O.route(lg, bias, K=8, C=C, block=32, rscale=2.5)
        bt, bw = brute_route(lg, bias, 8, C, 32, 2.5)
        np.testing.assert_array_equal(topk, bt)
        np.testing.assert_allclose(topw, bw, rtol=2e-6)


def test_router_logits_vs_fp64():
    x = gen.normal(70, (5, 2048)).astype(np.float32)
    Wr = (gen.normal(71, (2048, 256)) * 0.02).astype(np.float32)
    ref = x.astype(np.float64) @ Wr.astype(np.float64)
    out = O.router_logits(x, Wr)
    bound = 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(Wr).astype(np.float64))
    assert (np.abs(out - ref) <= bound).all()


# ---- dispatch (engine/ops.cu:333-423) --------------------------------------------------------------------------
def test_dispatch_invariants():
    T, E, K = 37, 256, 8
    topk = gen.distinct_rows(80, T, E, K)
    topw = gen.uniform(81, (T, K)).astype(np.float32)
    d = O.dispatch(topk, topw, E, True)
    assert d["count"].sum() == T * K and (d["start"] == np.concatenate([[0], np.cumsum(d["count"])[:-1]])).all()
    seen = set()
    for e in range(E):
        toks = d["slot_token"][d["start"][e]:d["start"][e] + d["count"][e]]
        assert (np.diff(toks) > 0).all()                            # token ascending within an expert
        for t in toks:
            seen.add((int(t), e))
    assert seen == {(t, int(e)) for t in range(T) for e in topk[t]}
    for t in range(T):
        for k in range(K):
            sl = d["tok_slots"][t, k]
            assert d["slot_token"][sl] == t and d["slot_weight"][sl] == topw[t, k]
            assert sl >= d["start"][topk[t, k]] and sl < d["start"][topk[t, k]] + d["count"][topk[t, k]]
        assert d["tok_slots"][t, K] == T * K + t and d["slot_token"][T * K + t] == t
        assert d["slot_weight"][T * K + t] == 1.0


# ---- integer core (engine/moe_i8.cu:1-14,162-169) --------------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_group_products_brute_force(bits):
    c, _, z = gen.matrix(90 + bits, 48, 512, bits)
    xq = np.clip(np.rint(gen.normal(91, (512,)) * 40), -127, 127).astype(np.int8)
    xq[:128] = 127                                                   # the bound: extreme codes and activations
    xsum = xq.reshape(4, 128).astype(np.int32).sum(1)
    P = O.group_products(c, z, xq, xsum)
    w = c.astype(np.int64) - np.repeat(z, 128, 1).astype(np.int64)
    ref = (w * xq.astype(np.int64)).reshape(48, 4, 128).sum(-1)
    np.testing.assert_array_equal(P, ref)


# ---- numerics primitives ---------------------------------------------------------------------------------------
def test_exp_sigmoid_silu_accuracy():
    xs = np.concatenate([gen.uniform(100, (4000,), -87, 88), [0.0, -0.0, 1e-30, -1e-30, 88.7, -103.0, -200.0]])
    for x in xs:
        x = float(np.float32(x))
        ref = math.exp(x)
        got = O.exp(x)
        if ref < 1.2e-38:                                            # subnormal / underflow region
            assert abs(got - ref) <= 2e-45 * 4
        else:
            assert abs(got - ref) <= 2.5 * np.spacing(np.float32(ref)), x
        s = 1.0 / (1.0 + math.exp(-x)) if x > -700 else 0.0
        assert abs(O.sigmoid(x) - s) <= 3e-7 * max(s, 1e-30) + 1e-45
        # SiLU feeds an fp16 rounding (2^-11): degree-5 exp and a Newton reciprocal, within 5e-6; clamped exp
        # argument below g = -80 (results under 1e-30)
        assert abs(O.silu(x) - x * s) <= 5e-6 * abs(x * s) + 1e-30, x     # measured max 3.5e-6 over [-90, 110]
    assert O.exp(89.0) == math.inf


def test_f32_to_f16_matches_numpy_rne():
    vals = np.concatenate([gen.normal(110, (20000,)).astype(np.float32) * np.float32(300),
                           gen.normal(111, (5000,)).astype(np.float32) * np.float32(1e-5),
                           np.array([65504, 65519.99, 65520, 1e9, -1e9, 6e-8, 2.98e-8, 0.0, -0.0, np.inf, -np.inf],
                                    np.float32)])
    # exact ties: values halfway between two fp16 numbers
    h = np.arange(1, 3000, dtype=np.uint16).view(np.float16).astype(np.float32)
    h2 = np.arange(2, 3001, dtype=np.uint16).view(np.float16).astype(np.float32)
    vals = np.concatenate([vals, (h + h2) / 2, -(h + h2) / 2,
                           np.arange(0x3c00, 0x3e00, dtype=np.uint16).view(np.float16).astype(np.float32) +
                           np.float32(2.0 ** -11)])
    got = np.array([O.f32_to_f16(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, vals.astype(np.float16).view(np.uint16))


# ---- the whole expert stage ------------------------------------------------------------------------------------
def _fixture_layer():
    mats, x, idx, w = gen.moe_case()
    M = gen.MOE
    blobs, gu_off, d_off, off = [], [], [], 0
    perm = O.gu_row_perm(M["I"])
    for e, ((cg, sg, zg), (cd, sd, zd)) in enumerate(mats):
        b = M["bits"][e]
        g = O.pack_i8(cg[perm], sg[perm], zg[perm], b)
        d = O.pack_i8(cd, sd, zd, b)
        gu_off.append(off); blobs.append(g); off += g.size
        d_off.append(off); blobs.append(d); off += d.size
    layer = dict(blob=np.concatenate(blobs), gu_off=np.array(gu_off, np.uint64), d_off=np.array(d_off, np.uint64),
                 bits=np.array(M["bits"], np.int8), H=M["H"], I=M["I"], E=M["E"], shared=False)
    return layer, x, idx, w, blobs


def test_experts_match_reference_gen_moe_case():
    f = fixture("moe_case.npz")
    layer, x, idx, w, blobs = _fixture_layer()
    assert str(f["digest"]) == gen.digest(x, idx, w)
    keys = sorted([f"gu{e}" for e in range(4)] + [f"d{e}" for e in range(4)])
    named = {f"gu{e}": blobs[2 * e] for e in range(4)} | {f"d{e}": blobs[2 * e + 1] for e in range(4)}
    assert str(f["blob_digest"]) == gen.digest(*[named[k] for k in keys]), "pack differs from packlib"
    L = O.Layer(layer, K=gen.MOE["K"])
    xq, xs, xsum = O.quant_a8(x)
    out = L.experts(xq, xs, xsum, idx, w)["out"]
    ref = f["acc"].astype(np.float64)
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    assert rel < 5e-3, rel                           # the reference's own bar (engine/tests/test_moe_i8.cu:173)
    err = np.abs(out - ref).max() / np.abs(ref).max()
    assert err <= 1e-3, err                          # the contract's max-abs 1e-3 relative
    assert err <= 1e-5, err                          # what the fixture pins (measured 2.2e-7)
    f64 = L.reference_f64(x, idx, w)
    assert np.linalg.norm(f64 - ref) / np.linalg.norm(ref) < 5e-3
    assert np.abs(f64 - ref).max() / np.abs(ref).max() <= 1e-5


def test_experts_vs_fp64_with_shared():
    layer = synth.make_layer(5, E=64, mix="mixed", shared=True)
    x = synth.make_x(6, 8, outlier_frac=0.01)
    L = O.Layer(layer)
    r = L.forward(x, C=48)
    f64 = L.reference_f64(x, r["topk"], r["topw"])
    assert np.linalg.norm(r["out"] - f64) / np.linalg.norm(f64) < 5e-3
    # every fp stage at max-abs 1e-3 relative against fp64 from the integer data the stage before produced
    check_stages_f64(layer, r["xq"], r["xs"], r["topk"], r["topw"], r["tok_slots"], r["Z"], r["zq"], r["zs"],
                     r["out"], range(8))
    # combine is the fixed-order sum of the weighted slot outputs
    acc = np.zeros_like(r["out"])
    for k in range(9):
        acc = acc + r["Y"][r["tok_slots"][:, k]]
    np.testing.assert_array_equal(acc, r["out"])


# ---- combine + un-rotation + residual + next-layer norm / rotation / A8 (engine/ops.cu:507-549) ---------------
def _sylvester(n):
    H = np.ones((1, 1))
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def test_combine_norm_closed_form():
    T, K1 = 3, 9
    Y = gen.normal(120, (T * K1, 2048)).astype(np.float32)
    tok_slots = np.arange(T * K1, dtype=np.int32).reshape(T, K1)[:, ::-1].copy()   # any slot order
    signs = np.where(gen.uniform(121, (2048,)) < 0.5, -1.0, 1.0).astype(np.float32)
    h = (gen.normal(122, (T, 2048)) * 3).astype(np.float32)
    eps = 1e-6
    hn, q, s, sm = O.combine_norm(Y, tok_slots, 9, signs, eps, h)
    H = _sylvester(2048)
    x = Y.astype(np.float64)[tok_slots].sum(1)
    h64 = h + (x @ H) * signs / np.sqrt(2048)                          # x Q^T, Q = diag(signs) H / sqrt(2048)
    np.testing.assert_allclose(hn, h64, rtol=0, atol=2e-6 * np.abs(h64).max())
    y64 = ((hn.astype(np.float64) / np.sqrt((hn.astype(np.float64) ** 2).mean(1, keepdims=True) + eps)) * signs) @ H
    y64 /= np.sqrt(2048)
    s64 = np.abs(y64.reshape(T, 16, 128)).max(-1) / 127
    np.testing.assert_allclose(s, s64, rtol=1e-5)
    qd = np.rint(y64.reshape(T, 16, 128) / s[:, :, None])
    assert np.abs(q.reshape(T, 16, 128) - qd).max() <= 1                  # rounding-boundary flips only
    assert (q.reshape(T, 16, 128) == qd).mean() > 0.999
    np.testing.assert_array_equal(sm, q.reshape(T, 16, 128).astype(np.int32).sum(-1))
    # the rotation is orthogonal: ||Q^T v|| = ||v|| (checked on the un-rotation increment)
    inc = (hn - h).astype(np.float64)
    np.testing.assert_allclose(np.linalg.norm(inc, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)


# ---- dense W.A8 projection (engine/engine.cu:380-383, :425, :434; KAT engine/tests/gen_dense_case.py) -------
@pytest.mark.parametrize("bits", [4, 8])
def test_dense_against_reference(bits):
    f = fixture("dense_case.npz")
    c, s, z, x = gen.dense_case(bits)
    assert gen.digest(c, s, z, x) == str(f[f"in_digest{bits}"])
    R, K = c.shape
    blob = O.pack_i8(c, s, z, bits)
    assert gen.digest(blob) == str(f[f"blob_digest{bits}"])        # same bytes as the reference's packlib
    xq, xs, xsum = O.quant_a8(x)
    y = O.dense(blob, R, K, bits, xq, xs, xsum)
    ref = f[f"ref{bits}"]                                            # A8(x) @ dequant(W)^T in fp32 (numpy)
    # the exact value of the same sum, in fp64
    xd = (xq.astype(np.float64).reshape(-1, K // 128, 128) * xs.astype(np.float64)[:, :, None]).reshape(-1, K)
    wd = (c.astype(np.float64) - np.repeat(z, 128, -1)) * np.repeat(s.astype(np.float64), 128, -1)
    exact = xd @ wd.T
    scale = np.abs(exact).max()
    assert np.abs(y - exact).max() <= 2e-6 * scale                  # one fp32 rounding per group
    assert np.abs(ref - exact).max() <= 2e-6 * scale
    assert np.abs(y - ref).max() <= 1e-3 * scale                     # the parity bar
    # accumulate: y0 + epilogue, one fp32 add per element
    y0 = gen.normal(3100, y.shape).astype(np.float32)
    np.testing.assert_array_equal(O.dense(blob, R, K, bits, xq, xs, xsum, y=y0), y0 + y)


def test_experts_from_z_reproduces_the_expert_stage():
    """orc_experts_from_z on the Z of orc_experts gives the same A8, slot outputs and combine, bit for bit."""
    layer = synth.make_layer(8, E=64, mix="mixed", shared=True)
    x = synth.make_x(3, 8)
    r = O.Layer(layer).forward(x, C=64)
    rz = O.Layer(layer).experts_from_z(r["Z"], r["topk"], r["topw"])
    for k in ("zq", "zs", "zsum", "Y", "out"):
        np.testing.assert_array_equal(np.asarray(rz[k]).view(np.uint8), np.asarray(r[k]).view(np.uint8), err_msg=k)


def test_experts_from_z_half_slot_outputs():
    """y_half: the slot outputs are the exact ones rounded to fp16 (numpy's round to nearest even) and the combine is
    the fixed-order fp32 sum of those; the output stays within the contract's 1e-3 of the exact one."""
    layer = synth.make_layer(8, E=64, mix="mixed", shared=True)
    x = synth.make_x(3, 8)
    r = O.Layer(layer).forward(x, C=64)
    rh = O.Layer(layer).experts_from_z(r["Z"], r["topk"], r["topw"], y_half=True)
    np.testing.assert_array_equal(rh["Y"].view(np.uint32),
                                  r["Y"].astype(np.float16).astype(np.float32).view(np.uint32))
    acc = np.zeros_like(rh["out"])
    for k in range(9):
        acc = acc + rh["Y"][r["tok_slots"][:, k]]
    np.testing.assert_array_equal(acc.view(np.uint32), rh["out"].view(np.uint32))
    err = np.abs(rh["out"] - r["out"]).max() / np.abs(r["out"]).max()
    assert 0 < err <= 1e-3, err
