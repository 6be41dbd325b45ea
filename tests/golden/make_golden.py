#!/usr/bin/env python3
"""Writes tests/golden/*.npz by calling the reference's own Python (packlib.py, the helpers of
engine/tests/gen_moe_case.py, route() of quant/s03_teacher_pass.py) on the deterministic inputs of gen.py.
Runs only where the reference tree is present (REF_ROOT, default /root/reference); the tests read the fixtures,
never the reference. Functions used:
  quant/packlib.py:167-197 pack_matrix_i8, :98-102 gu_row_perm
  engine/tests/gen_moe_case.py:20-36 dequant / a8 / hadamard, :77-93 the per-slot reference loop (restated
      here around those helpers, since main() needs model files)
  quant/s03_teacher_pass.py:132-146 route (with a duck-typed gate)
  engine/tests/gen_dense_case.py:20-25 the dense reference Y = A8(x) @ dequant(W)^T (restated around the helpers,
      since the script parses arguments and writes files)"""
from __future__ import annotations

import os
import sys
import types
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import gen  # noqa: E402

REF = Path(os.environ.get("REF_ROOT", "/root/reference"))
sys.path.insert(0, str(REF / "quant"))
sys.path.insert(0, str(REF / "engine" / "tests"))
import packlib as PL  # noqa: E402
import gen_moe_case as GM  # noqa: E402


def packlib_fixture():
    out = {}
    for b in (2, 3, 4, 8):
        c, s, z = gen.pack_case(b)
        out[f"blob{b}"] = PL.pack_matrix_i8(c, s, z, b)
        out[f"digest{b}"] = np.array(gen.digest(c, s, z))
    out["gu_row_perm512"] = np.asarray(PL.gu_row_perm(512), np.int32)
    np.savez_compressed(HERE / "packlib_i8.npz", **out)


def a8_fwht_fixture():
    rows = gen.a8_rows()
    v = gen.fwht_rows()
    np.savez_compressed(HERE / "a8_fwht.npz", a8_in_digest=np.array(gen.digest(rows)), a8_out=GM.a8(rows),
                        fwht_in_digest=np.array(gen.digest(v)), fwht_out=(v @ GM.hadamard(512)).astype(np.float32))


def route_fixture():
    import torch
    import s03_teacher_pass as S3
    logits, bias = gen.route_case()
    out = {"digest": np.array(gen.digest(logits, bias))}
    for C in (48, 256):
        # F.linear(h, W) with h = I (64 x 64) and W = logits^T returns the logits exactly.
        gate = types.SimpleNamespace(weight=torch.from_numpy(logits.T.copy()), expert_bias=torch.from_numpy(bias),
                                     block_size=32, expert_capacity=C, top_k=8, routed_scaling_factor=2.5)
        topk, w, pool = S3.route(gate, torch.eye(64))
        out[f"topk{C}"] = topk.numpy().astype(np.int32)
        out[f"topw{C}"] = w.numpy().astype(np.float32)
        out[f"pool{C}"] = pool.numpy().astype(np.int32)
    np.savez_compressed(HERE / "route.npz", **out)


def moe_fixture():
    mats, x, idx, w = gen.moe_case()
    I = gen.MOE["I"]
    W = [(GM.dequant(*gu), GM.dequant(*d)) for gu, d in mats]
    H512 = GM.hadamard(I)
    xf = GM.a8(x)
    T, K = idx.shape
    acc = np.zeros((T, x.shape[1]), np.float32)
    for t in range(T):                      # engine/tests/gen_moe_case.py:85-93 with fmt "i8"
        for k in range(K):
            gu, d = W[int(idx[t, k])]
            h = gu @ xf[t]
            z = (h[:I] / (1 + np.exp(-h[:I]))) * h[I:]
            z = z.astype(np.float16).astype(np.float32) @ H512
            acc[t] += w[t, k] * (d @ GM.a8(z))
    blobs = {}
    perm = PL.gu_row_perm(I)
    for e, ((cg, sg, zg), (cd, sd, zd)) in enumerate(mats):
        b = gen.MOE["bits"][e]
        blobs[f"gu{e}"] = PL.pack_matrix_i8(cg[perm], sg[perm], zg[perm], b)
        blobs[f"d{e}"] = PL.pack_matrix_i8(cd, sd, zd, b)
    np.savez_compressed(HERE / "moe_case.npz", acc=acc, digest=np.array(gen.digest(x, idx, w)),
                        blob_digest=np.array(gen.digest(*[blobs[k] for k in sorted(blobs)])))


def dense_fixture():
    out = {}
    for b in (4, 8):
        c, s, z, x = gen.dense_case(b)
        Wd = (c.astype(np.float32) - np.repeat(z, 128, -1)) * np.repeat(s.astype(np.float32), 128, -1)
        out[f"ref{b}"] = (GM.a8(x) @ Wd.T).astype(np.float32)
        out[f"blob_digest{b}"] = np.array(gen.digest(PL.pack_matrix_i8(c, s, z, b)))
        out[f"in_digest{b}"] = np.array(gen.digest(c, s, z, x))
    np.savez_compressed(HERE / "dense_case.npz", **out)


if __name__ == "__main__":
    dense_fixture()
    packlib_fixture()
    a8_fwht_fixture()
    route_fixture()
    moe_fixture()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
