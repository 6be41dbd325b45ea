"""Seeded synthetic MoE layers and inputs at the benchmark shapes (packlib format "i8", quant/packlib.py:140-197).

Uniformly random code bytes decode to uniformly random codes in any bit layout, so a matrix is generated
directly as packed tiles: random code bytes, then each tile's 48 bytes of group parameters (16 fp16 scales, 16 u8
zeros). Weight statistics follow the benchmark configurations: routed experts with scale ~U(0.005, 0.02) and zero
~U{0 .. 2^b - 1}; the W8A8 shared expert symmetric (zero 128) with one fp16 scale per output channel.
"""
from __future__ import annotations

import numpy as np

GROUP = 128
TILE_W = {2: 512, 3: 768, 4: 1024, 8: 2048}
MIXED_P = (0.61, 0.34, 0.06)      # shipped 2/3/4-bit allocation shares


def tile_bytes(bits: int) -> int:
    return TILE_W[bits] + 48


def matrix_bytes(R: int, K: int, bits: int) -> int:
    return (R // 16) * (K // GROUP) * tile_bytes(bits)


def expert_bytes(bits: int, H: int = 2048, I: int = 512) -> int:
    return matrix_bytes(2 * I, H, bits) + matrix_bytes(H, I, bits)


def random_matrix(rng: np.random.Generator, R: int, K: int, bits: int, *, scale=(0.005, 0.02),
                  per_row_scale: bool = False, symmetric: bool = False) -> np.ndarray:
    ns, nt = R // 16, K // GROUP
    wb = TILE_W[bits]
    m = np.empty((ns, nt, wb + 48), np.uint8)
    m[..., :wb] = np.frombuffer(rng.bytes(ns * nt * wb), np.uint8).reshape(ns, nt, wb)
    if per_row_scale:
        s = np.broadcast_to(rng.uniform(scale[0], scale[1], (ns, 1, 16)), (ns, nt, 16))
    else:
        s = rng.uniform(scale[0], scale[1], (ns, nt, 16))
    m[..., wb:wb + 32] = np.ascontiguousarray(s.astype(np.float16)).view(np.uint8).reshape(ns, nt, 32)
    if symmetric:
        m[..., wb + 32:] = 1 << (bits - 1)
    else:
        m[..., wb + 32:] = rng.integers(0, 1 << bits, (ns, nt, 16), dtype=np.uint8)
    return m.reshape(-1)


W8_SCALE = (0.005 / 16, 0.02 / 16)   # W8 codes span 16x the 4-bit range: keep the output scale comparable


def draw_bits(rng: np.random.Generator, E: int, mix) -> np.ndarray:
    if mix == "mixed":
        p = np.asarray(MIXED_P, np.float64)
        return rng.choice(np.array([2, 3, 4], np.int8), size=E, p=p / p.sum()).astype(np.int8)
    return np.full(E, int(mix), np.int8)


def make_layer(seed: int, *, E: int = 256, H: int = 2048, I: int = 512, mix="mixed", shared: bool = False,
               router: bool = True, zero_bias: bool = False, experts=None, w8_symmetric: bool = True) -> dict:
    """A layer as the reference stores it: blob + gu_off/d_off/bits ([E + shared]) + router Wr [H, E] + bias.

    experts: optional iterable of expert indices to materialise (others alias expert 0's matrices); tests use it
    to keep CPU-side work small while keeping E = 256 routing.
    w8_symmetric: routed 8-bit experts in the W8A8 convention of the shared expert (per-row fp16 scales at 1/16 of
    the 4-bit range, zero 128); False draws them like the narrower widths (random zeros: exercises the zero term,
    but the products grow 16x and may overflow fp16 Z on large activations)."""
    rng = np.random.default_rng(seed)
    bits = draw_bits(rng, E, mix)
    Wr = (rng.standard_normal((H, E), dtype=np.float32) * np.float32(0.02)) if router else None
    bias = np.zeros(E, np.float32) if zero_bias else rng.uniform(-0.1, 0.1, E).astype(np.float32)
    n = E + (1 if shared else 0)
    gu_off = np.zeros(n, np.uint64)
    d_off = np.zeros(n, np.uint64)
    bits_all = np.zeros(n, np.int8)
    bits_all[:E] = bits
    chunks, off = [], 0
    want = set(range(E)) if experts is None else set(int(e) for e in experts) | {0}
    first = {}
    for e in range(E):
        b = int(bits[e])
        if e not in want:
            if b not in first:
                want.add(e)
            else:
                gu_off[e], d_off[e] = first[b]
                continue
        if b == 8 and w8_symmetric:
            g = random_matrix(rng, 2 * I, H, 8, scale=W8_SCALE, per_row_scale=True, symmetric=True)
            d = random_matrix(rng, H, I, 8, scale=W8_SCALE, per_row_scale=True, symmetric=True)
        else:
            g = random_matrix(rng, 2 * I, H, b)
            d = random_matrix(rng, H, I, b)
        gu_off[e] = off; chunks.append(g); off += g.size
        d_off[e] = off; chunks.append(d); off += d.size
        first.setdefault(b, (gu_off[e], d_off[e]))
    if shared:
        bits_all[E] = 8
        g = random_matrix(rng, 2 * I, H, 8, scale=W8_SCALE, per_row_scale=True, symmetric=True)
        d = random_matrix(rng, H, I, 8, scale=W8_SCALE, per_row_scale=True, symmetric=True)
        gu_off[E] = off; chunks.append(g); off += g.size
        d_off[E] = off; chunks.append(d); off += d.size
    return {"blob": np.concatenate(chunks), "gu_off": gu_off, "d_off": d_off, "bits": bits_all, "Wr": Wr,
            "bias": bias, "E": E, "H": H, "I": I, "shared": shared}


def touched_weight_bytes(layer: dict, topk: np.ndarray) -> int:
    """Weight-stream bytes of one pass: every expert some token routes to, once, plus the shared expert."""
    E = layer["E"]
    used = np.unique(np.asarray(topk).reshape(-1))
    tot = sum(expert_bytes(int(layer["bits"][e]), layer["H"], layer["I"]) for e in used)
    if layer["shared"]:
        tot += expert_bytes(8, layer["H"], layer["I"])
    return int(tot)


def make_x(seed: int, T: int, H: int = 2048, outlier_frac: float = 0.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H), dtype=np.float32)
    if outlier_frac > 0:
        ch = rng.choice(H, max(1, int(round(H * outlier_frac))), replace=False)
        x[:, ch] *= np.float32(20.0)
    return x


def logits_zipf(seed: int, T: int, E: int = 256, s: float = 1.1) -> np.ndarray:
    """Router logits whose top-8 (after sigmoid, zero bias) follow Zipf(s) expert popularity: Gumbel-top-k
    sampling without replacement with p_e proportional to rank^-s over a random expert order."""
    rng = np.random.default_rng(seed)
    rank = rng.permutation(E) + 1
    logp = -s * np.log(rank.astype(np.float64))
    g = rng.gumbel(size=(T, E))
    return (logp[None, :] + g).astype(np.float32)


def logits_skewed(seed: int, T: int, E: int = 256, K: int = 8, hot: int = 16) -> np.ndarray:
    """Logits whose top-K puts K/2 picks per token on `hot` experts (so they receive 50% of slots)."""
    rng = np.random.default_rng(seed)
    hot_set = rng.choice(E, hot, replace=False)
    cold_set = np.setdiff1d(np.arange(E), hot_set)
    lg = (rng.standard_normal((T, E)) - 4.0).astype(np.float32)
    for t in range(T):
        a = rng.choice(hot_set, K // 2, replace=False)
        b = rng.choice(cold_set, K - K // 2, replace=False)
        lg[t, a] = 4.0 + 0.1 * rng.standard_normal(K // 2)
        lg[t, b] = 4.0 + 0.1 * rng.standard_normal(K - K // 2)
    return lg


def bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def write_model_dir(path, layer: dict, li: int = 1, signs=None, extra_cfg=None) -> dict:
    """Write `layer` in the reference's model-directory format (quant/s07_pack_experts.py, s07b, s07c_index.py):
    engine.idx, experts_L<li>.bin (routed experts at their blob offsets), nonexpert_L<li>.bin (the shared expert's
    gate_up / down, 4 KiB aligned) and small.bin (router bf16 [E, H], expert bias, signs). Returns the layer as
    the loader should see it (router rounded to bf16)."""
    from pathlib import Path
    p = Path(path)
    p.mkdir(parents=True, exist_ok=True)
    E, H, I = layer["E"], layer["H"], layer["I"]
    blob = layer["blob"]
    # routed experts: the blob up to the shared expert's first matrix
    end = int(min(layer["gu_off"][E], layer["d_off"][E])) if layer["shared"] else blob.size
    (p / f"experts_L{li}.bin").write_bytes(blob[:end].tobytes())
    lines = [f"C hidden_size {H}", f"C moe_intermediate_size {I}", f"C num_experts {E}", "C num_experts_per_tok 8",
             "C expert_capacity 48", "C block_size 32", "C routed_scaling_factor 2.5", "C nonexpert_bits 8"]
    lines += [f"C {k} {v}" for k, v in (extra_cfg or {}).items()]
    lines.append(f"F experts_L{li}.bin {end}")
    for e in range(E):
        lines.append(f"E {li} {e} {int(layer['bits'][e])} {int(layer['gu_off'][e])} {int(layer['d_off'][e])}")

    def align(f, off):
        pad = (-off) % 4096
        f.write(b"\0" * pad)
        return off + pad

    if layer["shared"]:
        gu = blob[int(layer["gu_off"][E]):int(layer["gu_off"][E]) + matrix_bytes(2 * I, H, 8)]
        dn = blob[int(layer["d_off"][E]):int(layer["d_off"][E]) + matrix_bytes(H, I, 8)]
        with open(p / f"nonexpert_L{li}.bin", "wb") as f:
            off = 0
            for name, arr, shape in (("gate_up", gu, (2 * I, H)), ("down", dn, (H, I))):
                off = align(f, off)
                f.write(arr.tobytes())
                lines.append(f"T nonexpert_L{li}.bin {name} {off} {arr.size} i8tiles8 {shape[0]} {shape[1]}")
                off += arr.size
    wr = bf16_round(layer["Wr"])
    if signs is None:
        signs = np.where(np.random.default_rng(li).random(H) < 0.5, -1.0, 1.0).astype(np.float32)
    with open(p / "small.bin", "wb") as f:
        off = 0
        for name, arr, dt in ((f"L{li}.router", (np.ascontiguousarray(wr.T).view(np.uint32) >> 16).astype(np.uint16), "bf16"),
                              (f"L{li}.expert_bias", layer["bias"].astype(np.float32), "f32"),
                              ("signs", np.asarray(signs, np.float32), "f32")):
            off = align(f, off)
            f.write(np.ascontiguousarray(arr).tobytes())
            shape = " ".join(str(s) for s in arr.shape)
            lines.append(f"T small.bin {name} {off} {arr.nbytes} {dt} {shape}")
            off += arr.nbytes
    (p / "engine.idx").write_text("\n".join(lines) + "\n")
    return dict(layer, Wr=wr, signs=np.asarray(signs, np.float32))
