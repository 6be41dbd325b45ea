"""C-ABI checks that need no GPU: the library loads, exports every function include/llmoe.h declares, and
rejects bad layer descriptions before touching the device."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import llmoe
from llmoe import synth

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "llmoe.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(llmoe_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not llmoe.LIB_PATH.exists():
        pytest.skip("libllmoe.so not built (python -c 'import __graft_entry__ as g; g.build()')")
    return llmoe.load_library()


def test_header_and_binding_agree():
    assert declared() == sorted(llmoe.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared():
        assert hasattr(lib, name), name


def _create(desc_kw, bits=None, blob_bytes=None):
    d = llmoe.LayerDesc(hidden=2048, inter=512, n_experts=64, top_k=8, pool=48, block=32, routed_scale=2.5,
                        has_shared=0, max_tokens=32)
    for k, v in desc_kw.items():
        setattr(d, k, v)
    E = d.n_experts + d.has_shared
    bits = np.full(max(E, 1), 2, np.int8) if bits is None else bits
    eb = synth.expert_bytes(2)
    gu = np.arange(max(E, 1), dtype=np.uint64) * np.uint64(eb)
    dd = gu + np.uint64(synth.matrix_bytes(1024, 2048, 2))
    blob = np.zeros(16, np.uint8)
    nbytes = eb * E if blob_bytes is None else blob_bytes
    bias = np.zeros(max(E, 1), np.float32)
    out = ctypes.c_void_p()
    rc = llmoe.load_library().llmoe_layer_create(ctypes.byref(d), blob.ctypes.data, ctypes.c_size_t(nbytes),
                                                 gu.ctypes.data, dd.ctypes.data, bits.ctypes.data, None,
                                                 bias.ctypes.data, ctypes.byref(out))
    return rc, llmoe.load_library().llmoe_last_error().decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(hidden=1024), "hidden"), (dict(inter=256), "inter"), (dict(n_experts=100), "n_experts"),
    (dict(top_k=9), "top_k"), (dict(pool=4), "pool"), (dict(block=64), "block"), (dict(max_tokens=0), "max_tokens"),
])
def test_create_rejects_bad_desc(lib, kw, msg):
    rc, err = _create(kw)
    assert rc == llmoe.LLMOE_EINVAL and msg in err


def test_create_rejects_bad_bits_and_short_blob(lib):
    bits = np.full(64, 2, np.int8)
    bits[7] = 5
    rc, err = _create({}, bits=bits)
    assert rc == llmoe.LLMOE_EINVAL and "expert 7" in err
    rc, err = _create({}, blob_bytes=1000)
    assert rc == llmoe.LLMOE_EINVAL and "beyond the blob" in err


# ---- the model-directory loader (engine/engine.cu:54-75, quant/s07c_index.py) ------------------------------
def _load(path, layer=1):
    h = ctypes.c_void_p()
    rc = llmoe.load_library().llmoe_layer_load(str(path).encode(), layer, 64, ctypes.byref(h))
    return rc, llmoe.load_library().llmoe_last_error().decode()


def test_load_missing_dir(lib, tmp_path):
    rc, err = _load(tmp_path / "nope")
    assert rc == llmoe.LLMOE_EINVAL and "engine.idx" in err


def test_load_rejects_bad_index(lib, tmp_path):
    L = synth.make_layer(3, E=64, experts=[0], shared=True)
    synth.write_model_dir(tmp_path, L, li=2)
    idx = (tmp_path / "engine.idx").read_text()
    rc, err = _load(tmp_path, layer=5)
    assert rc == llmoe.LLMOE_EINVAL and "layer 5" in err
    (tmp_path / "engine.idx").write_text(idx.replace("E 2 7 ", "E 2 7 0 ", 1).replace("E 2 7 0 " + idx.split("E 2 7 ")[1].split()[0] + " ", "E 2 7 0 ", 1))
    rc, err = _load(tmp_path, layer=2)
    assert rc == llmoe.LLMOE_EINVAL and "pruned" in err
    (tmp_path / "engine.idx").write_text(idx + "X what\n")
    rc, err = _load(tmp_path, layer=2)
    assert rc == llmoe.LLMOE_EINVAL and "unknown record" in err
    (tmp_path / "engine.idx").write_text(idx.replace(f"F experts_L2.bin ", "F experts_L2.bin 1", 1))
    rc, err = _load(tmp_path, layer=2)
    assert rc == llmoe.LLMOE_EINVAL and "engine.idx says" in err


def test_model_signs(lib, tmp_path):
    L = synth.make_layer(4, E=64, experts=[0], shared=True)
    ref = synth.write_model_dir(tmp_path, L, li=1)
    out = np.zeros(2048, np.float32)
    assert llmoe.load_library().llmoe_model_signs(str(tmp_path).encode(), out.ctypes.data, 2048) == 0
    np.testing.assert_array_equal(out, ref["signs"])


def test_dense_create_rejects(lib):
    """llmoe_dense_create validates its shape and blob before any GPU work."""
    h = ctypes.c_void_p()
    blob = np.zeros(16, np.uint8)
    for rows, k, bits in ((512, 1024, 8), (100, 2048, 8), (512, 2048, 5)):
        rc = lib.llmoe_dense_create(rows, k, bits, blob.ctypes.data, blob.nbytes, 32, ctypes.byref(h))
        assert rc == llmoe.LLMOE_EINVAL, (rows, k, bits)
    rc = lib.llmoe_dense_create(512, 2048, 8, blob.ctypes.data, blob.nbytes, 32, ctypes.byref(h))
    assert rc == llmoe.LLMOE_EINVAL and "blob" in lib.llmoe_last_error().decode()


# every entry point that takes a layer, called with a null one: LLMOE_EINVAL and a message, no device call
_NULL_LAYER_CALLS = {
    "llmoe_route": lambda f: f(None, None, None, 32, None),
    "llmoe_dispatch": lambda f: f(None, None, None, 32, None),
    "llmoe_experts": lambda f: f(None, None, None, None, 32, None, None),
    "llmoe_experts_norm": lambda f: f(None, None, None, None, 32, None, ctypes.c_float(1e-6), None, None, None, None,
                                      None),
    "llmoe_experts_scratch": lambda f: f(None, None, None, None, 32, None, None),
    "llmoe_layer_forward": lambda f: f(None, None, None, 32, None, None),
    "llmoe_layer_forward_norm": lambda f: f(None, None, None, 32, None, ctypes.c_float(1e-6), None, None, None, None,
                                            None),
    "llmoe_layer_set_numerics": lambda f: f(None, 0),
    "llmoe_layer_set_profiling": lambda f: f(None, 1),
    "llmoe_layer_buffers": lambda f: f(None, ctypes.byref(llmoe.Buffers())),
    "llmoe_layer_weight_bytes": lambda f: f(None, ctypes.byref(ctypes.c_size_t())),
}


@pytest.mark.parametrize("name", sorted(_NULL_LAYER_CALLS))
def test_null_layer_rejected(lib, name):
    rc = _NULL_LAYER_CALLS[name](getattr(lib, name))
    assert rc == -1, f"{name} returned {rc}"   # LLMOE_EINVAL
    assert b"null layer" in lib.llmoe_last_error(), lib.llmoe_last_error()
