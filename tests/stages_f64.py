"""Stage-wise fp64 checks of the expert stage at the contract's tolerance (max-abs 1e-3 relative).

An end-to-end comparison with an independent fp64 path re-quantises Z' on its own, and a code that flips at an
A8 rounding boundary moves an output element by one quantisation step (about 4e-3 of the group maximum), so the
end-to-end bar can only be relative L2 (the reference's own, engine/tests/test_moe_i8.cu:173). Each fp stage is
checked here against fp64 from the integer data the previous stage actually produced:

- gate_up epilogue + SiLU: Z against fp16(SiLU(g) u) with g, u = dequant(W_gu) @ dequant(A8(x)) in fp64
  (engine/tests/gen_moe_case.py:81-85): max-abs <= 1e-3 relative (fp16 rounding alone is 2^-11 of each value);
- FWHT-512 + A8: dequant(Z') against the fp64 FWHT of Z / sqrt(512) (gen_moe_case.py:86-87): every element within
  half a quantisation step of its group plus 1e-5 of the row's largest value for the fp32 butterflies (the A8
  bound, which a wrong butterfly or scale breaks);
- down epilogue, routing weight and combine: out[t] against sum_k w_k dequant(W_d) @ dequant(Z'_slot) in fp64
  (gen_moe_case.py:88): max-abs <= 1e-3 relative.

Inputs are numpy arrays as llmoe / the oracle produce them; only the given tokens are checked (the fp64 matrices of
every expert they touch are built).
"""
import numpy as np

import oracle

TOL = 1e-3


def _sylvester512():
    H = np.ones((1, 1))
    while H.shape[0] < 512:
        H = np.block([[H, H], [H, -H]])
    return H / np.sqrt(512.0)


def _dequant(codes, scale, zero):
    return (codes.astype(np.float64) - np.repeat(zero.astype(np.float64), 128, -1)) * \
        np.repeat(scale.astype(np.float64), 128, -1)


def check_stages_f64(L, xq, xs, topk, topw, tok_slots, Z, zq, zs, out, tokens, tol=TOL):
    """L: synth layer dict; xq/xs: the A8 of x; topk/topw: routing; tok_slots [T, K+1]; Z (fp16 bits) / zq / zs
    [S, ...]; out [T, H]. Raises AssertionError with the stage that fails. Returns the three measured errors."""
    H, I, E = L["H"], L["I"], L["E"]
    K = topk.shape[1]
    perm = oracle.gu_row_perm(I)
    Hd = _sylvester512()
    mats = {}

    def expert(e):
        if e not in mats:
            b = int(L["bits"][e])
            go, do = int(L["gu_off"][e]), int(L["d_off"][e])
            c, s, z = oracle.unpack_i8(L["blob"][go:go + oracle.matrix_bytes(2 * I, H, b)], 2 * I, H, b)
            gu = np.empty((2 * I, H))
            gu[perm] = _dequant(c, s, z)           # packed row p is logical row perm[p]
            c, s, z = oracle.unpack_i8(L["blob"][do:do + oracle.matrix_bytes(H, I, b)], H, I, b)
            mats[e] = (gu, _dequant(c, s, z))
        return mats[e]

    errs = {"Z": 0.0, "fwht": 0.0, "out": 0.0}
    zmax = omax = 0.0
    zerr = oerr = 0.0
    for t in tokens:
        xd = np.repeat(xs[t].astype(np.float64), 128) * xq[t].astype(np.float64)
        acc = np.zeros(H)
        for k in range(K + (1 if L["shared"] else 0)):
            e, w = (int(topk[t, k]), float(topw[t, k])) if k < K else (E, 1.0)
            s = int(tok_slots[t, k])
            gu, dn = expert(e)
            h = gu @ xd
            g, u = h[:I], h[I:]
            zref = g / (1.0 + np.exp(-g)) * u
            zg = Z[s].view(np.float16).astype(np.float64)
            zerr = max(zerr, float(np.abs(zg - zref).max()))
            zmax = max(zmax, float(np.abs(zref).max()))
            v = Hd @ zg                              # FWHT of the slot's own Z (H symmetric)
            step = np.repeat(zs[s].astype(np.float64), 128)
            dq = zq[s].astype(np.float64) * step
            # half a step, plus the fp32 butterflies' rounding (about 1e-7 of the row's largest value)
            excess = np.abs(dq - v) - 0.5 * step
            assert excess.max() <= 1e-5 * np.abs(v).max(), \
                f"token {t} slot {s}: FWHT + A8 beyond half a step ({excess.max():.3e})"
            errs["fwht"] = max(errs["fwht"], float((np.abs(dq - v) / step).max()))
            acc += w * (dn @ dq)
        oerr = max(oerr, float(np.abs(out[t].astype(np.float64) - acc).max()))
        omax = max(omax, float(np.abs(acc).max()))
    errs["Z"] = zerr / max(zmax, 1e-30)
    errs["out"] = oerr / max(omax, 1e-30)
    assert errs["Z"] <= tol, f"gate_up epilogue: max-abs rel {errs['Z']:.3e} > {tol}"
    assert errs["out"] <= tol, f"down + combine: max-abs rel {errs['out']:.3e} > {tol}"
    return errs
