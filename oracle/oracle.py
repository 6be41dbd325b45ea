"""ctypes wrapper of the CPU oracle (libmoe_oracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker (or the timed CPU baseline); the product path (libllmoe.so) never calls it.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libmoe_oracle.so"

_lib = None


class OrcLayer(ctypes.Structure):
    _fields_ = [("H", ctypes.c_int), ("I", ctypes.c_int), ("E", ctypes.c_int), ("K", ctypes.c_int),
                ("has_shared", ctypes.c_int), ("blob", ctypes.c_void_p), ("gu_off", ctypes.c_void_p),
                ("d_off", ctypes.c_void_p), ("bits", ctypes.c_void_p)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} not built (make -C oracle)")
        L = ctypes.CDLL(str(LIB))
        vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.orc_exp.argtypes = [f]; L.orc_exp.restype = f
        L.orc_sigmoid.argtypes = [f]; L.orc_sigmoid.restype = f
        L.orc_silu.argtypes = [f]; L.orc_silu.restype = f
        L.orc_f32_to_f16.argtypes = [f]; L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]; L.orc_f16_to_f32.restype = f
        L.orc_matrix_bytes.argtypes = [i, i, i]; L.orc_matrix_bytes.restype = ctypes.c_size_t
        L.orc_pack_i8.argtypes = [vp, vp, vp, i, i, i, vp]
        L.orc_unpack_i8.argtypes = [vp, i, i, i, vp, vp, vp]
        L.orc_gu_row_perm.argtypes = [i, vp]
        L.orc_quant_a8.argtypes = [vp, i, i, vp, vp, vp]
        L.orc_router_logits.argtypes = [vp, vp, i, i, i, vp]
        L.orc_route.argtypes = [vp, vp, i, i, i, i, i, f, vp, vp]
        L.orc_dispatch.argtypes = [vp, vp, i, i, i, i, vp, vp, vp, vp, vp]
        L.orc_dispatch.restype = i
        L.orc_group_products.argtypes = [vp, vp, i, i, vp, vp, vp]
        L.orc_fwht_a8.argtypes = [vp, i, vp, vp, vp]
        L.orc_fwht512_f32.argtypes = [vp]
        L.orc_experts.argtypes = [ctypes.POINTER(OrcLayer), vp, vp, vp, i, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                  vp, i]
        L.orc_experts.restype = i
        L.orc_experts_from_z.argtypes = [ctypes.POINTER(OrcLayer), vp, i, i, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i]
        L.orc_experts_from_z.restype = i
        L.orc_reference_f64.argtypes = [ctypes.POINTER(OrcLayer), vp, i, vp, vp, vp, i]
        L.orc_reference_f64.restype = i
        L.orc_combine_norm.argtypes = [vp, vp, i, i, i, vp, f, vp, vp, vp, vp]
        L.orc_dense.argtypes = [vp, i, i, i, vp, vp, vp, i, vp, i, i]
        L.orc_dense.restype = i
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---- primitives -------------------------------------------------------------------------------------------
def exp(x: float) -> float: return lib().orc_exp(x)
def sigmoid(x: float) -> float: return lib().orc_sigmoid(x)
def silu(x: float) -> float: return lib().orc_silu(x)
def f32_to_f16(x: float) -> int: return lib().orc_f32_to_f16(x)


def matrix_bytes(R, K, bits) -> int:
    return int(lib().orc_matrix_bytes(R, K, bits))


def pack_i8(codes, scale, zero, bits):
    R, K = codes.shape
    out = np.zeros(matrix_bytes(R, K, bits), np.uint8)
    lib().orc_pack_i8(_p(np.ascontiguousarray(codes, np.uint8)),
                      _p(np.ascontiguousarray(np.asarray(scale, np.float16).view(np.uint16))),
                      _p(np.ascontiguousarray(zero, np.uint8)), R, K, bits, _p(out))
    return out


def unpack_i8(blob, R, K, bits):
    codes = np.zeros((R, K), np.uint8)
    scale = np.zeros((R, K // 128), np.uint16)
    zero = np.zeros((R, K // 128), np.uint8)
    lib().orc_unpack_i8(_p(np.ascontiguousarray(blob, np.uint8)), R, K, bits, _p(codes), _p(scale), _p(zero))
    return codes, scale.view(np.float16), zero


def gu_row_perm(I):
    p = np.zeros(2 * I, np.int32)
    lib().orc_gu_row_perm(I, _p(p))
    return p


def quant_a8(x):
    x = np.ascontiguousarray(x, np.float32)
    R, K = x.shape
    q = np.zeros((R, K), np.int8)
    s = np.zeros((R, K // 128), np.float32)
    sm = np.zeros((R, K // 128), np.int32)
    lib().orc_quant_a8(_p(x), R, K, _p(q), _p(s), _p(sm))
    return q, s, sm


def router_logits(x, Wr):
    x = np.ascontiguousarray(x, np.float32)
    Wr = np.ascontiguousarray(Wr, np.float32)
    T, H = x.shape
    E = Wr.shape[1]
    out = np.zeros((T, E), np.float32)
    lib().orc_router_logits(_p(x), _p(Wr), T, H, E, _p(out))
    return out


def route(logits, bias, K=8, C=256, block=32, rscale=2.5):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    topk = np.zeros((T, K), np.int32)
    topw = np.zeros((T, K), np.float32)
    lib().orc_route(_p(logits), _p(np.ascontiguousarray(bias, np.float32)), T, E, K, C, block, rscale, _p(topk),
                    _p(topw))
    return topk, topw


def dispatch(topk, topw, E, has_shared):
    topk = np.ascontiguousarray(topk, np.int32)
    topw = np.ascontiguousarray(topw, np.float32)
    T, K = topk.shape
    S = T * K + (T if has_shared else 0)
    count = np.zeros(E, np.int32)
    start = np.zeros(E, np.int32)
    slot_token = np.zeros(S, np.int32)
    slot_weight = np.zeros(S, np.float32)
    tok_slots = np.zeros((T, K + 1), np.int32)
    lib().orc_dispatch(_p(topk), _p(topw), T, E, K, int(has_shared), _p(count), _p(start), _p(slot_token),
                       _p(slot_weight), _p(tok_slots))
    return dict(count=count, start=start, slot_token=slot_token, slot_weight=slot_weight, tok_slots=tok_slots)


def group_products(codes, zero, xq, xsum):
    codes = np.ascontiguousarray(codes, np.uint8)
    R, K = codes.shape
    P = np.zeros((R, K // 128), np.int32)
    lib().orc_group_products(_p(codes), _p(np.ascontiguousarray(zero, np.uint8)), R, K,
                             _p(np.ascontiguousarray(xq, np.int8)), _p(np.ascontiguousarray(xsum, np.int32)), _p(P))
    return P


def fwht512(v):
    v = np.array(v, np.float32, copy=True)
    lib().orc_fwht512_f32(_p(v))
    return v


def fwht_a8(Z):
    Z = np.ascontiguousarray(Z, np.uint16)
    n = Z.shape[0]
    q = np.zeros((n, 512), np.int8)
    s = np.zeros((n, 4), np.float32)
    sm = np.zeros((n, 4), np.int32)
    lib().orc_fwht_a8(_p(Z), n, _p(q), _p(s), _p(sm))
    return q, s, sm


def combine_norm(Y, tok_slots, nk, signs, eps, h):
    """-> (h_new, q, s, sum): combine of the nk first slots of each token, FWHT-2048 un-rotation with signs,
    residual add into a copy of h, then the next layer's RMSNorm + rotation + A8."""
    Y = np.ascontiguousarray(Y, np.float32)
    tok_slots = np.ascontiguousarray(tok_slots, np.int32)
    T, K1 = tok_slots.shape
    hn = np.array(h, np.float32, copy=True)
    q = np.zeros((T, 2048), np.int8)
    s = np.zeros((T, 16), np.float32)
    sm = np.zeros((T, 16), np.int32)
    lib().orc_combine_norm(_p(Y), _p(tok_slots), T, nk, K1, _p(np.ascontiguousarray(signs, np.float32)), eps, _p(hn),
                           _p(q), _p(s), _p(sm))
    return hn, q, s, sm


def dense(blob, R, K, bits, xq, xs, xsum, y=None, nthreads=0):
    """Dense W.A8 projection of the A8 rows (xq, xs, xsum) by the [R, K] packlib-i8 matrix: y = epilogue(P), or,
    with y given, y + epilogue(P) (a new array)."""
    blob = np.ascontiguousarray(blob, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    T = xq.shape[0]
    out = np.zeros((T, R), np.float32) if y is None else np.array(y, np.float32, copy=True)
    rc = lib().orc_dense(_p(blob), R, K, bits, _p(xq), _p(np.ascontiguousarray(xs, np.float32)),
                         _p(np.ascontiguousarray(xsum, np.int32)), T, _p(out), 0 if y is None else 1, nthreads)
    if rc:
        raise RuntimeError(f"orc_dense: {rc}")
    return out


class Layer:
    """Oracle view of a synthetic layer dict (llmoe.synth.make_layer)."""

    def __init__(self, layer: dict, K: int = 8):
        self.layer = layer
        self.blob = np.ascontiguousarray(layer["blob"], np.uint8)
        self.gu_off = np.ascontiguousarray(layer["gu_off"], np.uint64)
        self.d_off = np.ascontiguousarray(layer["d_off"], np.uint64)
        self.bits = np.ascontiguousarray(layer["bits"], np.int8)
        self.K = K
        self.c = OrcLayer(layer["H"], layer["I"], layer["E"], K, int(layer["shared"]), _p(self.blob),
                          _p(self.gu_off), _p(self.d_off), _p(self.bits))

    def experts(self, xq, xs, xsum, topk, topw, nthreads=0):
        """Full expert stage -> dict(out, Y, Z, zq, zs, zsum, dispatch arrays)."""
        L = self.layer
        H, I, E = L["H"], L["I"], L["E"]
        T = topk.shape[0]
        dsp = dispatch(topk, topw, E, L["shared"])
        S = dsp["slot_token"].size
        Z = np.zeros((S, I), np.uint16)
        zq = np.zeros((S, I), np.int8)
        zs = np.zeros((S, 4), np.float32)
        zsum = np.zeros((S, 4), np.int32)
        Y = np.zeros((S, H), np.float32)
        out = np.zeros((T, H), np.float32)
        rc = lib().orc_experts(ctypes.byref(self.c), _p(np.ascontiguousarray(xq, np.int8)),
                               _p(np.ascontiguousarray(xs, np.float32)), _p(np.ascontiguousarray(xsum, np.int32)), T,
                               _p(dsp["count"]), _p(dsp["start"]), _p(dsp["slot_token"]), _p(dsp["slot_weight"]),
                               _p(dsp["tok_slots"]), _p(Z), _p(zq), _p(zs), _p(zsum), _p(Y), _p(out), nthreads)
        if rc != 0:
            raise RuntimeError(f"orc_experts failed: {rc}")
        return dict(out=out, Y=Y, Z=Z, zq=zq, zs=zs, zsum=zsum, **dsp)

    def experts_from_z(self, Z, topk, topw, nthreads=0, y_half=False):
        """The expert stage after gate_up, from given fp16 Z [S, I] bits: FWHT-512 + A8, down, combine. y_half: the
        slot outputs Y rounded to fp16 (nearest even) before the combine, as the build's fast numerics store them
        (Y is returned as fp32 holding those fp16 values)."""
        L = self.layer
        H, I, E = L["H"], L["I"], L["E"]
        T = topk.shape[0]
        dsp = dispatch(topk, topw, E, L["shared"])
        S = dsp["slot_token"].size
        Z = np.ascontiguousarray(Z, np.uint16).reshape(S, I)
        zq = np.zeros((S, I), np.int8)
        zs = np.zeros((S, 4), np.float32)
        zsum = np.zeros((S, 4), np.int32)
        Y = np.zeros((S, H), np.float32)
        out = np.zeros((T, H), np.float32)
        rc = lib().orc_experts_from_z(ctypes.byref(self.c), _p(Z), int(y_half), T, _p(dsp["count"]), _p(dsp["start"]),
                                      _p(dsp["slot_token"]), _p(dsp["slot_weight"]), _p(dsp["tok_slots"]), _p(zq),
                                      _p(zs), _p(zsum), _p(Y), _p(out), nthreads)
        if rc != 0:
            raise RuntimeError(f"orc_experts_from_z failed: {rc}")
        return dict(out=out, Y=Y, zq=zq, zs=zs, zsum=zsum, **dsp)

    def reference_f64(self, x, topk, topw, nthreads=0):
        T = x.shape[0]
        out = np.zeros((T, self.layer["H"]), np.float64)
        rc = lib().orc_reference_f64(ctypes.byref(self.c), _p(np.ascontiguousarray(x, np.float32)), T,
                                     _p(np.ascontiguousarray(topk, np.int32)),
                                     _p(np.ascontiguousarray(topw, np.float32)), _p(out), nthreads)
        if rc != 0:
            raise RuntimeError(f"orc_reference_f64 failed: {rc}")
        return out

    def forward(self, x, logits=None, C=256, block=32, rscale=2.5, nthreads=0):
        """A8 -> route (x Wr or given logits) -> experts."""
        L = self.layer
        xq, xs, xsum = quant_a8(x)
        lg = router_logits(x, L["Wr"]) if logits is None else np.ascontiguousarray(logits, np.float32)
        topk, topw = route(lg, L["bias"], self.K, C, block, rscale)
        r = self.experts(xq, xs, xsum, topk, topw, nthreads)
        r.update(xq=xq, xs=xs, xsum=xsum, logits=lg, topk=topk, topw=topw)
        return r
