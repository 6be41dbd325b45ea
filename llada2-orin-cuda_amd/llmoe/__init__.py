"""Python binding of libllmoe (include/llmoe.h): the LLaDA2 routed-expert MoE layer on MI355X.

The compute path is the HIP library libllmoe.so next to this file (built by `python -m llmoe.build` or
`__graft_entry__.build()`); this module only marshals arguments. There is no fallback: if the library is not
built, loading fails loudly.

Device memory and streams come from PyTorch (torch.cuda tensors and torch.cuda.current_stream()); every call
passes raw device pointers through the C ABI, as the reference's server binds its engine through ctypes
(server/server.py:62-71 of patrickbdevaney/llada2-orin-cuda).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libllmoe.so"

LLMOE_OK = 0
SCRATCH_MAX_TOKENS = 64   # LLMOE_SCRATCH_MAX_TOKENS of include/llmoe.h
NUMERICS_EXACT, NUMERICS_FAST = 0, 1
LLMOE_EINVAL = -1   # bad argument or shape
LLMOE_ENOMEM = -2
LLMOE_EHIP = -3
LLMOE_ESTATE = -4


class LLMoEError(RuntimeError):
    pass


class LayerDesc(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int),
        ("inter", ctypes.c_int),
        ("n_experts", ctypes.c_int),
        ("top_k", ctypes.c_int),
        ("pool", ctypes.c_int),
        ("block", ctypes.c_int),
        ("routed_scale", ctypes.c_float),
        ("has_shared", ctypes.c_int),
        ("max_tokens", ctypes.c_int),
    ]


class Buffers(ctypes.Structure):
    _fields_ = [
        ("xq", ctypes.c_void_p), ("xs", ctypes.c_void_p), ("xsum", ctypes.c_void_p),
        ("logits_part", ctypes.c_void_p),
        ("topk", ctypes.c_void_p), ("topw", ctypes.c_void_p),
        ("count", ctypes.c_void_p), ("start", ctypes.c_void_p),
        ("slot_token", ctypes.c_void_p), ("slot_weight", ctypes.c_void_p),
        ("tok_slots", ctypes.c_void_p),
        ("items", ctypes.c_void_p), ("n_items", ctypes.c_void_p),
        ("Z", ctypes.c_void_p), ("zq", ctypes.c_void_p), ("zs", ctypes.c_void_p), ("zsum", ctypes.c_void_p),
        ("Y", ctypes.c_void_p),
        ("ntok", ctypes.c_int), ("max_items", ctypes.c_int),
    ]


EXPORTS = [
    "llmoe_layer_create", "llmoe_layer_destroy", "llmoe_quantize_a8", "llmoe_route", "llmoe_dispatch",
    "llmoe_experts", "llmoe_experts_norm", "llmoe_layer_forward", "llmoe_layer_buffers", "llmoe_layer_weight_bytes",
    "llmoe_group_products", "llmoe_layer_set_profiling", "llmoe_layer_stage_ms", "llmoe_layer_time_stage", "llmoe_layers_time_stage",
    "llmoe_layer_load", "llmoe_model_signs", "llmoe_dense_create", "llmoe_dense_destroy", "llmoe_dense_forward",
    "llmoe_last_error", "llmoe_experts_scratch", "llmoe_layer_set_numerics", "llmoe_selftest_f16",
    "llmoe_layer_forward_norm",
]

STAGES = ["quant", "router", "route", "dispatch", "gate_up", "fwht", "down", "combine"]

_lib = None


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libllmoe.so (raises if it is not built: the HIP path is the only path)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise LLMoEError(f"{p} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    lib = ctypes.CDLL(str(p))
    vp, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.llmoe_last_error.restype = ctypes.c_char_p
    lib.llmoe_layer_load.argtypes = [ctypes.c_char_p, i, i, ctypes.POINTER(ctypes.c_void_p)]
    lib.llmoe_model_signs.argtypes = [ctypes.c_char_p, vp, i]
    lib.llmoe_dense_create.argtypes = [i, i, i, vp, sz, i, ctypes.POINTER(ctypes.c_void_p)]
    lib.llmoe_dense_destroy.argtypes = [vp]
    lib.llmoe_dense_forward.argtypes = [vp, vp, vp, vp, i, vp, i, vp]
    lib.llmoe_layer_create.argtypes = [ctypes.POINTER(LayerDesc), vp, sz, vp, vp, vp, vp, vp,
                                       ctypes.POINTER(ctypes.c_void_p)]
    lib.llmoe_layer_destroy.argtypes = [vp]
    lib.llmoe_quantize_a8.argtypes = [vp, i, i, vp, vp, vp, vp]
    lib.llmoe_route.argtypes = [vp, vp, vp, i, vp]
    lib.llmoe_dispatch.argtypes = [vp, vp, vp, i, vp]
    lib.llmoe_experts.argtypes = [vp, vp, vp, vp, i, vp, vp]
    lib.llmoe_experts_scratch.argtypes = [vp, vp, vp, vp, i, vp, vp]
    lib.llmoe_experts_norm.argtypes = [vp, vp, vp, vp, i, vp, f, vp, vp, vp, vp, vp]
    lib.llmoe_layer_forward.argtypes = [vp, vp, vp, i, vp, vp]
    lib.llmoe_layer_forward_norm.argtypes = [vp, vp, vp, i, vp, f, vp, vp, vp, vp, vp]
    lib.llmoe_layer_buffers.argtypes = [vp, ctypes.POINTER(Buffers)]
    lib.llmoe_layer_weight_bytes.argtypes = [vp, ctypes.POINTER(sz)]
    lib.llmoe_group_products.argtypes = [vp, i, i, vp, vp, i, vp, vp]
    lib.llmoe_selftest_f16.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    lib.llmoe_layer_set_profiling.argtypes = [vp, i]
    lib.llmoe_layer_set_numerics.argtypes = [vp, i]
    lib.llmoe_layer_stage_ms.argtypes = [vp, ctypes.POINTER(ctypes.c_float)]
    lib.llmoe_layer_time_stage.argtypes = [vp, i, i, vp, ctypes.POINTER(ctypes.c_float)]
    lib.llmoe_layers_time_stage.argtypes = [ctypes.POINTER(ctypes.c_void_p), i, i, i, vp, ctypes.POINTER(ctypes.c_float)]
    for name in EXPORTS:
        if name != "llmoe_last_error":
            getattr(lib, name).restype = ctypes.c_int
    if path is None:
        _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != LLMOE_OK:
        msg = load_library().llmoe_last_error().decode(errors="replace")
        raise LLMoEError(f"libllmoe error {rc}: {msg}")


def _ptr(t) -> int | None:
    """Device (or host numpy) pointer of a tensor / array, None for None."""
    if t is None:
        return None
    if isinstance(t, np.ndarray):
        assert t.flags["C_CONTIGUOUS"]
        return t.ctypes.data
    assert t.is_contiguous(), "tensors passed to libllmoe must be contiguous"
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else stream


class Layer:
    """One MoE layer resident in HBM (llmoe_layer_*). Weights: packlib format "i8" blob + per-expert tables."""

    def __init__(self, blob: np.ndarray, gu_off, d_off, bits, router_bias, router_w=None, *, hidden=2048, inter=512,
                 n_experts=256, top_k=8, pool=256, block=32, routed_scale=2.5, has_shared=False, max_tokens=4096):
        self.lib = load_library()
        self.desc = LayerDesc(hidden, inter, n_experts, top_k, pool, block, routed_scale, int(has_shared), max_tokens)
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        gu_off = np.ascontiguousarray(gu_off, dtype=np.uint64)
        d_off = np.ascontiguousarray(d_off, dtype=np.uint64)
        bits = np.ascontiguousarray(bits, dtype=np.int8)
        bias = np.ascontiguousarray(router_bias, dtype=np.float32)
        rw = None if router_w is None else np.ascontiguousarray(router_w, dtype=np.float32)
        h = ctypes.c_void_p()
        _check(self.lib.llmoe_layer_create(ctypes.byref(self.desc), _ptr(blob), blob.nbytes, _ptr(gu_off),
                                           _ptr(d_off), _ptr(bits), _ptr(rw), _ptr(bias), ctypes.byref(h)))
        self.handle = h
        self.T = None

    @classmethod
    def load(cls, model_dir, layer: int, max_tokens: int = 4096) -> "Layer":
        """llmoe_layer_load: the MoE half of `layer` from the reference's model directory."""
        self = cls.__new__(cls)
        self.lib = load_library()
        h = ctypes.c_void_p()
        _check(self.lib.llmoe_layer_load(str(model_dir).encode(), layer, max_tokens, ctypes.byref(h)))
        self.handle = h
        self.T = None
        self.desc = LayerDesc(2048, 512, 256, 8, 48, 32, 2.5, 1, max_tokens)   # informational
        return self

    def close(self) -> None:
        if getattr(self, "handle", None):
            _check(self.lib.llmoe_layer_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- calls (device tensors in, device tensors out) ----
    def forward(self, x, logits=None, out=None, stream=None):
        import torch
        T = x.shape[0]
        if out is None:
            out = torch.empty((T, self.desc.hidden), dtype=torch.float32, device=x.device)
        _check(self.lib.llmoe_layer_forward(self.handle, _ptr(x), _ptr(logits), T, _ptr(out), _stream(stream)))
        self.T = T
        return out

    def route(self, T, x=None, logits=None, stream=None):
        _check(self.lib.llmoe_route(self.handle, _ptr(x), _ptr(logits), T, _stream(stream)))
        self.T = T

    def dispatch(self, topk, topw, stream=None):
        T = topk.shape[0]
        _check(self.lib.llmoe_dispatch(self.handle, _ptr(topk), _ptr(topw), T, _stream(stream)))
        self.T = T

    def experts(self, xq, xs, xsum, out=None, stream=None):
        import torch
        T = xq.shape[0]
        if out is None:
            out = torch.empty((T, self.desc.hidden), dtype=torch.float32, device=xq.device)
        _check(self.lib.llmoe_experts(self.handle, _ptr(xq), _ptr(xs), _ptr(xsum), T, _ptr(out), _stream(stream)))
        return out

    def experts_scratch(self, xq, xs, xsum, out=None, stream=None):
        """llmoe_experts with the intermediates in the library's static per-GPU scratch (T <= 64)."""
        import torch
        T = xq.shape[0]
        if out is None:
            out = torch.empty((T, self.desc.hidden), dtype=torch.float32, device=xq.device)
        _check(self.lib.llmoe_experts_scratch(self.handle, _ptr(xq), _ptr(xs), _ptr(xsum), T, _ptr(out),
                                              _stream(stream)))
        return out

    def experts_norm(self, xq, xs, xsum, signs, eps, h, out=None, stream=None):
        """Experts, then un-rotation + residual into h (in place) + the next layer's RMSNorm / rotation / A8.
        Returns (q_next, s_next, sum_next), written into `out` when given."""
        import torch
        T = xq.shape[0]
        if out is None:
            out = (torch.empty((T, 2048), dtype=torch.int8, device=xq.device),
                   torch.empty((T, 16), dtype=torch.float32, device=xq.device),
                   torch.empty((T, 16), dtype=torch.int32, device=xq.device))
        q, s, sm = out
        _check(self.lib.llmoe_experts_norm(self.handle, _ptr(xq), _ptr(xs), _ptr(xsum), T, _ptr(signs), float(eps),
                                           _ptr(h), _ptr(q), _ptr(s), _ptr(sm), _stream(stream)))
        return q, s, sm

    def forward_norm(self, x, signs, eps, h, logits=None, out=None, stream=None):
        """The layer forward with the fused epilogue (llmoe_layer_forward_norm): h += the un-rotated MoE output (in
        place); returns the next layer's A8 (q_next, s_next, sum_next), written into `out` when given."""
        import torch
        T = x.shape[0]
        if out is None:
            out = (torch.empty((T, 2048), dtype=torch.int8, device=x.device),
                   torch.empty((T, 16), dtype=torch.float32, device=x.device),
                   torch.empty((T, 16), dtype=torch.int32, device=x.device))
        q, s, sm = out
        _check(self.lib.llmoe_layer_forward_norm(self.handle, _ptr(x), _ptr(logits), T, _ptr(signs), float(eps),
                                                 _ptr(h), _ptr(q), _ptr(s), _ptr(sm), _stream(stream)))
        self.T = T
        return q, s, sm

    def group_products(self, expert: int, which: int, xq, xsum, stream=None):
        import torch
        n, kw = xq.shape
        rows = 2 * self.desc.inter if which == 0 else self.desc.hidden
        P = torch.zeros((n, rows, kw // 128), dtype=torch.int32, device=xq.device)
        _check(self.lib.llmoe_group_products(self.handle, expert, which, _ptr(xq), _ptr(xsum), n, _ptr(P),
                                             _stream(stream)))
        return P

    def set_numerics(self, fast: bool) -> None:
        """LLMOE_NUMERICS_FAST (the gate_up SiLU by the hardware transcendentals) or LLMOE_NUMERICS_EXACT."""
        _check(self.lib.llmoe_layer_set_numerics(self.handle, NUMERICS_FAST if fast else NUMERICS_EXACT))

    def set_profiling(self, on: bool) -> None:
        _check(self.lib.llmoe_layer_set_profiling(self.handle, int(on)))

    def stage_ms(self) -> dict:
        """Per-stage milliseconds of the latest profiled call (stages not run: absent)."""
        arr = (ctypes.c_float * len(STAGES))()
        _check(self.lib.llmoe_layer_stage_ms(self.handle, arr))
        return {n: float(v) for n, v in zip(STAGES, arr) if v >= 0}

    def time_stage(self, stage: str, reps: int = 50, stream=None) -> float:
        """Average ms of one expert stage of the latest call, re-launched `reps` times back to back."""
        v = ctypes.c_float()
        _check(self.lib.llmoe_layer_time_stage(self.handle, STAGES.index(stage), reps, _stream(stream),
                                               ctypes.byref(v)))
        return float(v.value)

    def buffers(self) -> Buffers:
        b = Buffers()
        _check(self.lib.llmoe_layer_buffers(self.handle, ctypes.byref(b)))
        return b

    def weight_bytes(self) -> int:
        v = ctypes.c_size_t()
        _check(self.lib.llmoe_layer_weight_bytes(self.handle, ctypes.byref(v)))
        return int(v.value)

    def read(self, name: str, shape, dtype):
        """Copy a workspace buffer (llmoe_buffers field) to a numpy array (synchronises the device)."""
        import torch
        ptr = getattr(self.buffers(), name)
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        torch.cuda.synchronize()
        out = np.empty(shape, dtype=dtype)
        _hip_memcpy_d2h(out, ptr, n)
        return out


def quantize_a8(x, stream=None):
    """llmoe_quantize_a8 of a contiguous fp32 [rows, cols] device tensor: (q int8, s fp32 [rows, cols/128],
    sum int32 [rows, cols/128])."""
    import torch
    rows, cols = x.shape
    q = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    s = torch.empty((rows, cols // 128), dtype=torch.float32, device=x.device)
    sm = torch.empty((rows, cols // 128), dtype=torch.int32, device=x.device)
    _check(load_library().llmoe_quantize_a8(_ptr(x), rows, cols, _ptr(q), _ptr(s), _ptr(sm), _stream(stream)))
    return q, s, sm


class Dense:
    """A dense W.A8 projection [rows, 2048] resident in HBM (llmoe_dense_*), packlib "i8" blob."""

    def __init__(self, blob: np.ndarray, rows: int, bits: int, k: int = 2048, max_tokens: int = 4096):
        self.lib = load_library()
        self.rows, self.k = rows, k
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        h = ctypes.c_void_p()
        _check(self.lib.llmoe_dense_create(rows, k, bits, _ptr(blob), blob.nbytes, max_tokens, ctypes.byref(h)))
        self.handle = h

    def forward(self, xq, xs, xsum, out=None, accumulate: bool = False, stream=None):
        """y = W A8(x) (or out += that with accumulate): xq int8 [T, 2048], xs fp32 / xsum int32 [T, 16]."""
        import torch
        T = xq.shape[0]
        if out is None:
            out = torch.empty((T, self.rows), dtype=torch.float32, device=xq.device)
        _check(self.lib.llmoe_dense_forward(self.handle, _ptr(xq), _ptr(xs), _ptr(xsum), T, _ptr(out),
                                            int(accumulate), _stream(stream)))
        return out

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.llmoe_dense_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def selftest_f16() -> int:
    """llmoe_selftest_f16: the number of finite fp32 inputs on which the device's hardware fp16 conversion differs
    from round-to-nearest-even in integer ops (0 expected)."""
    n = ctypes.c_uint64()
    _check(load_library().llmoe_selftest_f16(ctypes.byref(n)))
    return int(n.value)


def time_stage_layers(layers, stage: str, reps: int = 20, stream=None) -> float:
    """Average ms per launch of one expert stage, re-launched over several layers in turn (llmoe_layers_time_stage)."""
    lib = load_library()
    arr = (ctypes.c_void_p * len(layers))(*[L.handle.value for L in layers])
    v = ctypes.c_float()
    _check(lib.llmoe_layers_time_stage(arr, len(layers), STAGES.index(stage), reps, _stream(stream), ctypes.byref(v)))
    return float(v.value)


_hip = None


def _hip_memcpy_d2h(dst: np.ndarray, src_ptr: int, nbytes: int) -> None:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
    rc = _hip.hipMemcpy(dst.ctypes.data, src_ptr, nbytes, 2)   # hipMemcpyDeviceToHost
    if rc != 0:
        raise LLMoEError(f"hipMemcpy D2H failed: {rc}")
