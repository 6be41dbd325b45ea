"""Deterministic inputs for the golden fixtures (splitmix64 streams, so the inputs never depend on a numpy
random-generator version). Both the fixture writer and the tests regenerate the same arrays from these
functions; the fixtures hold only the outputs and a checksum of the inputs."""
from __future__ import annotations

import hashlib

import numpy as np

_M = np.uint64(0xFFFFFFFFFFFFFFFF)


def u64(seed: int, n: int) -> np.ndarray:
    """splitmix64 outputs 1..n of the stream `seed` (Steele, Lea, Flood 2014)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15))
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, shape, lo=0.0, hi=1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u = (u64(seed, n) >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    return (lo + (hi - lo) * u).reshape(shape)


def normal(seed: int, shape) -> np.ndarray:
    """Irwin-Hall(12) - 6: mean 0, variance 1, bounded by +-6."""
    n = int(np.prod(shape))
    return uniform(seed, (n, 12)).sum(1).reshape(shape) - 6.0


def codes(seed: int, shape, bits: int) -> np.ndarray:
    return (u64(seed, int(np.prod(shape))) % np.uint64(1 << bits)).astype(np.uint8).reshape(shape)


def matrix(seed: int, R: int, K: int, bits: int):
    """(codes [R,K] u8 < 2^bits, scale [R,K/128] fp16 in [0.005, 0.02), zero [R,K/128] u8 < 2^bits)."""
    c = codes(seed, (R, K), bits)
    s = uniform(seed + 1, (R, K // 128), 0.005, 0.02).astype(np.float16)
    z = codes(seed + 2, (R, K // 128), bits)
    return c, s, z


def distinct_rows(seed: int, T: int, E: int, K: int) -> np.ndarray:
    """Per token K distinct experts of E (first K of a random permutation)."""
    keys = u64(seed, T * E).reshape(T, E)
    return np.argsort(keys, axis=1, kind="stable")[:, :K].astype(np.int32)


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


# ---- the cases ------------------------------------------------------------------------------------------
PACK_SHAPE = (32, 256)                 # R, K of the packlib fixtures
MOE = dict(E=4, bits=(2, 3, 4, 8), H=512, I=512, T=6, K=2)


def pack_case(bits: int):
    return matrix(100 + bits, *PACK_SHAPE, bits)


def a8_rows() -> np.ndarray:
    """Rows of 512 fp32 with the quantiser's edge cases: all zero, exact .5 ties, one outlier, subnormal scale,
    negative-only, values at +-max, and plain random rows."""
    rows = np.zeros((8, 512), np.float32)
    rows[1, :256] = np.arange(256, dtype=np.float32) * 0.5 - 63.5     # ties at x.5 with s = 1 per group max 127
    rows[1, 127] = 127.0
    rows[1, 255] = -127.0
    rows[1, 256:] = normal(7, 256)
    rows[2] = normal(8, 512) * 0.01
    rows[2, 300] = 40.0
    rows[3] = normal(9, 512) * 1e-39
    rows[4] = -np.abs(normal(10, 512))
    rows[5, ::2] = 3.0
    rows[5, 1::2] = -3.0
    rows[6] = normal(11, 512)
    rows[7] = normal(12, 512) * 100.0
    return rows


def fwht_rows() -> np.ndarray:
    v = normal(20, (4, 512)).astype(np.float32)
    v[0] = 0.0
    v[0, 5] = 1.0                      # e_5
    return v


def route_case():
    """64 tokens (2 blocks of 32) x 256 experts of tie-free logits and a bias ~U(-0.1, 0.1)."""
    logits = (normal(30, (64, 256)) * 1.5).astype(np.float32)
    bias = uniform(31, (256,), -0.1, 0.1).astype(np.float32)
    return logits, bias


DENSE = dict(R=512, K=2048, T=8)


def dense_case(bits: int):
    """A dense [R, K] matrix in the distribution of engine/tests/gen_dense_case.py (fp16 scales
    U(0.5, 1.5) * 2 / 2^b * 0.05, zeros within 2 of 2^b / 2) and T fp16-valued token rows."""
    R, K, T = DENSE["R"], DENSE["K"], DENSE["T"]
    c = codes(3000 + bits, (R, K), bits)
    s = (uniform(3001 + bits, (R, K // 128), 0.5, 1.5) * 2.0 / 2 ** bits * 0.05).astype(np.float16)
    z = (codes(3002 + bits, (R, K // 128), 2).astype(np.int32) + 2 ** bits // 2 - 2).astype(np.uint8)
    x = normal(3003 + bits, (T, K)).astype(np.float16).astype(np.float32)
    return c, s, z, x


def moe_case():
    """Tiny routed-expert layer in the format gen_moe_case.py builds: logical matrices per expert, tokens,
    routing, weights."""
    E, H, I, T, K = MOE["E"], MOE["H"], MOE["I"], MOE["T"], MOE["K"]
    mats = []
    for e, b in enumerate(MOE["bits"]):
        mats.append((matrix(1000 + 10 * e, 2 * I, H, b), matrix(1005 + 10 * e, H, I, b)))
    x = normal(40, (T, H)).astype(np.float16).astype(np.float32)
    x[1, 17] = 25.0                    # an outlier channel
    idx = distinct_rows(41, T, E, K)
    w = uniform(42, (T, K), 0.05, 0.6).astype(np.float32)
    return mats, x, idx, w
