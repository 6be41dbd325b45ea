"""GPU parity: libllmoe.so (HIP, gfx950) against the CPU oracle on the same seeded inputs.

The bar: integer outputs (A8 codes and sums, expert indices, slots, work items, int32 group products) bit-exact;
fp32 outputs (router logits, routing weights, SiLU -> fp16, FWHT + A8 scales, expert outputs, combine) bit-exact
as well, since both sides run the same fp32 operation sequence -- and, as the contract's floor, within max-abs
1e-3 relative (FP_TOL) of the oracle.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from llmoe import Layer, synth

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
sys.path.insert(0, str(Path(__file__).resolve().parent))
import gen  # noqa: E402
from stages_f64 import check_stages_f64  # noqa: E402

pytestmark = pytest.mark.gpu

FP_TOL = 1e-3   # max |gpu - oracle| <= FP_TOL * max |oracle|


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def close(gpu, ref, what):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref).max() if gpu.size else 0.0
    scale = max(np.abs(ref).max() if ref.size else 0.0, 1e-30)
    assert err <= FP_TOL * scale, f"{what}: max abs err {err} > {FP_TOL} * {scale}"


def make_gpu_layer(L, pool, max_tokens=256, K=8):
    return Layer(L["blob"], L["gu_off"], L["d_off"], L["bits"], L["bias"], L["Wr"], n_experts=L["E"], top_k=K,
                 pool=pool, has_shared=L["shared"], max_tokens=max_tokens)


_LAYERS = {}


def layer_for(mix, shared, seed=11):
    key = (mix, shared, seed)
    if key not in _LAYERS:
        _LAYERS[key] = synth.make_layer(seed, mix=mix, shared=shared, w8_symmetric=False)
    return _LAYERS[key]


# ------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("rows", [1, 7, 64])
def test_quant_a8_bit_exact(gpu, rows):
    import torch
    import llmoe
    say(f"[quant_a8] rows={rows}")
    x = synth.make_x(100 + rows, rows, 2048, outlier_frac=0.01)
    x[0, :128] = 0.0                       # an all-zero group: scale floor 1e-30
    q_ref, s_ref, sum_ref = oracle.quant_a8(x)
    xd = to_dev(x, gpu)
    q = torch.empty((rows, 2048), dtype=torch.int8, device=gpu)
    s = torch.empty((rows, 16), dtype=torch.float32, device=gpu)
    sm = torch.empty((rows, 16), dtype=torch.int32, device=gpu)
    lib = llmoe.load_library()
    rc = lib.llmoe_quantize_a8(xd.data_ptr(), rows, 2048, q.data_ptr(), s.data_ptr(), sm.data_ptr(),
                               torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(sm.cpu().numpy(), sum_ref)


def test_fwht_stage_fused_at_decode(gpu):
    """One routing block: FWHT-512 + A8 runs inside the streamed down GEMM, so re-launching the FWHT stage alone is
    refused (its time is in the down stage); with several blocks the standalone FWHT kernel re-launches."""
    import torch
    import llmoe
    say("[fwht stage] T=32 and T=64")
    L = layer_for("mixed", True)
    G = make_gpu_layer(L, 256)
    run_layer(G, synth.make_x(70, 32), gpu)
    with pytest.raises(llmoe.LLMoEError, match="fused into the down GEMM"):
        G.time_stage("fwht", reps=2)
    assert G.time_stage("down", reps=2) > 0
    run_layer(G, synth.make_x(71, 64), gpu)
    assert G.time_stage("fwht", reps=2) > 0
    torch.cuda.synchronize()
    G.close()


def test_hw_f16_conversion_is_round_to_nearest_even(gpu):
    """The kernels round fp32 -> fp16 with v_cvt_f16_f32; the CPU checker restates round-to-nearest-even in integer
    ops (pinned against numpy in the CPU suite). Every finite fp32 bit pattern gives the same bits both ways."""
    import llmoe
    say("[f16 self-test] all 2^32 patterns")
    assert llmoe.selftest_f16() == 0


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("which", [0, 1])
def test_group_products_bit_exact(gpu, bits, which):
    """Exact int32 P_g = sum code*xq - zero*Sxq for every (token, row, group), through relayout + MFMA."""
    say(f"[group_products] bits={bits} which={which}")
    L = synth.make_layer(31 + bits, mix=bits, experts=[5], w8_symmetric=False)
    G = make_gpu_layer(L, 256)
    e = 5
    R, Kw = (1024, 2048) if which == 0 else (2048, 512)
    off = int(L["gu_off"][e] if which == 0 else L["d_off"][e])
    codes, scale, zero = oracle.unpack_i8(L["blob"][off:off + synth.matrix_bytes(R, Kw, bits)], R, Kw, bits)
    rng = np.random.default_rng(7)
    n = 37
    xq = rng.integers(-127, 128, (n, Kw), dtype=np.int8)
    xq[0] = 127
    xq[1] = -127
    xsum = xq.reshape(n, -1, 128).astype(np.int32).sum(-1).astype(np.int32)
    P = G.group_products(e, which, to_dev(xq, gpu), to_dev(xsum, gpu)).cpu().numpy()
    for i in range(n):
        ref = oracle.group_products(codes, zero, xq[i], xsum[i])
        assert np.array_equal(P[i], ref), f"token {i}: {np.argwhere(P[i] != ref)[:5]}"
    G.close()


def run_layer(G, x, dev, logits=None):
    import torch
    out = G.forward(to_dev(x, dev), None if logits is None else to_dev(logits, dev))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check_full(G, r, T, K, shared, tokens=None):
    """Compare every stage of the GPU workspace with the oracle run r (optionally only some tokens)."""
    H, I = 2048, 512
    S = T * K + (T if shared else 0)
    topk = G.read("topk", (T, K), np.int32)
    topw = G.read("topw", (T, K), np.float32)
    assert np.array_equal(topk, r["topk"]), "expert indices differ"
    assert np.array_equal(topw.view(np.uint32), r["topw"].view(np.uint32)), "routing weights differ"
    assert np.array_equal(G.read("slot_token", (S,), np.int32), r["slot_token"])
    assert np.array_equal(G.read("slot_weight", (S,), np.float32), r["slot_weight"])
    ts = G.read("tok_slots", (T, K + 1), np.int32)
    assert np.array_equal(ts, r["tok_slots"])
    E = r["count"].size
    assert np.array_equal(G.read("count", (E,), np.int32), r["count"])
    Z = G.read("Z", (S, I), np.uint16)
    zq = G.read("zq", (S, I), np.int8)
    zs = G.read("zs", (S, 4), np.float32)
    zsum = G.read("zsum", (S, 4), np.int32)
    Y = G.read("Y", (S, H), np.float32)
    if tokens is None:
        slots = np.arange(S)
    else:
        slots = np.unique(ts[tokens][:, :K + (1 if shared else 0)].reshape(-1))
    for name, a, b in (("Z", Z, r["Z"]), ("zq", zq, r["zq"]), ("zsum", zsum, r["zsum"])):
        assert np.array_equal(a[slots], b[slots]), f"{name} differs at slots {np.argwhere((a[slots] != b[slots]).any(-1))[:5].ravel()}"
    close(zs[slots], r["zs"][slots], "zs")
    assert np.array_equal(zs[slots].view(np.uint32), r["zs"][slots].view(np.uint32)), "zs not bit-exact"
    close(Y[slots], r["Y"][slots], "Y")
    assert np.array_equal(Y[slots].view(np.uint32), r["Y"][slots].view(np.uint32)), "Y not bit-exact"


@pytest.mark.parametrize("T,mix,shared,pool", [
    (32, 4, False, 48),          # config 0: 4-bit, block pool 48
    (32, 4, False, 256),         # config 0 without the pool
    (32, "mixed", True, 256),    # config 1
    (1, "mixed", True, 256),
    (45, "mixed", True, 48),     # ragged last block
    (96, 8, True, 256),
    (200, "mixed", True, 48),    # tiled units for the shared expert and the pool's busiest experts
    (33, "mixed", True, 256),    # the first T over one routing block: a second block of one token
    (64, 2, False, 48),          # exactly two blocks
    (256, "mixed", True, 256),   # T = the layer's max_tokens
])
def test_layer_forward_matches_oracle(gpu, T, mix, shared, pool):
    say(f"[layer] T={T} mix={mix} shared={shared} pool={pool}")
    L = layer_for(mix, shared)
    G = make_gpu_layer(L, pool)
    x = synth.make_x(1000 + T, T)
    out = run_layer(G, x, gpu)
    r = oracle.Layer(L).forward(x, C=pool)
    assert np.array_equal(G.read("xq", (T, 2048), np.int8), r["xq"])
    check_full(G, r, T, 8, shared)
    close(out, r["out"], "out")
    assert np.array_equal(out.view(np.uint32), r["out"].view(np.uint32)), "combine not bit-exact"
    ref64 = oracle.Layer(L).reference_f64(x, r["topk"], r["topw"])
    assert np.linalg.norm(out - ref64) / np.linalg.norm(ref64) < 5e-3   # engine/tests/test_moe_i8.cu:173
    # each fp stage of the GPU's own data at max-abs 1e-3 relative against fp64 (gate_up epilogue + SiLU, FWHT + A8,
    # down + combine)
    S = T * 8 + (T if shared else 0)
    check_stages_f64(L, G.read("xq", (T, 2048), np.int8), G.read("xs", (T, 16), np.float32), r["topk"], r["topw"],
                     G.read("tok_slots", (T, 9), np.int32), G.read("Z", (S, 512), np.uint16),
                     G.read("zq", (S, 512), np.int8), G.read("zs", (S, 4), np.float32), out,
                     sorted({0, T // 2, T - 1}))
    G.close()


@pytest.mark.parametrize("E,K,T,pool", [
    (64, 4, 32, 16),      # decode, pool
    (128, 6, 32, 256),    # decode, no pool
    (64, 8, 100, 48),     # several routing blocks, tiled experts
    (128, 2, 200, 256),
    (192, 8, 32, 48),     # 24 decode expert slices (3 per XCD), 3 wide router tiles
    (192, 8, 70, 256),
])
def test_other_expert_counts(gpu, E, K, T, pool):
    """The ABI's other shapes (E a multiple of 64 up to 256, top_k <= 8): every stage bit-exact."""
    say(f"[shape] E={E} K={K} T={T} pool={pool}")
    L = synth.make_layer(900 + E + K, E=E, mix="mixed", shared=True)
    G = make_gpu_layer(L, pool, max_tokens=256, K=K)
    x = synth.make_x(950 + T, T)
    out = run_layer(G, x, gpu)
    r = oracle.Layer(L, K=K).forward(x, C=pool)
    check_full(G, r, T, K, True)
    assert np.array_equal(out.view(np.uint32), r["out"].view(np.uint32)), "combine not bit-exact"
    G.close()


def _decode_state(G, T, K, E, shared):
    """Every buffer a decode step writes, as numpy arrays (the gate_up unit list up to its count)."""
    S = T * K + (T if shared else 0)
    n = G.read("n_items", (4,), np.int32)
    st = {"n_items": n, "items": G.read("items", (int(n[0]), 4), np.int32)}
    for name, shape, dt in (("topk", (T, K), np.int32), ("topw", (T, K), np.float32), ("count", (E,), np.int32),
                            ("start", (E,), np.int32), ("slot_token", (S,), np.int32),
                            ("slot_weight", (S,), np.float32), ("tok_slots", (T, K + 1), np.int32),
                            ("Z", (S, 512), np.uint16), ("zq", (S, 512), np.int8), ("zs", (S, 4), np.float32),
                            ("zsum", (S, 4), np.int32), ("Y", (S, 2048), np.float32)):
        st[name] = G.read(name, shape, dt)
    return st


@pytest.mark.parametrize("E,K,T,pool,mix,shared", [
    (256, 8, 32, 256, "mixed", True),   # config 1
    (256, 8, 32, 48, 4, False),         # config 0 (pool)
    (256, 8, 1, 256, "mixed", True),
    (256, 8, 17, 48, "mixed", True),    # two shared items, pool
    (64, 4, 32, 16, "mixed", True),
    (128, 6, 5, 256, 8, False),
])
def test_decode_forward_plans_like_dispatch(gpu, E, K, T, pool, mix, shared):
    """A decode layer forward plans the slots inside its gate_up GEMM (no dispatch kernel): every buffer, the gate_up
    unit list and the output equal those of route + experts (the dispatch kernel's plan), bit for bit; a re-launch of
    the gate_up stage from the written list reproduces Z; and a second forward (the down GEMM cleared the routing
    masks) matches a fresh route + experts again."""
    import torch
    say(f"[decode plan] E={E} K={K} T={T} pool={pool} mix={mix} shared={shared}")
    L = synth.make_layer(700 + E + K + T, E=E, mix=mix, shared=shared)
    x = [synth.make_x(720 + T + i, T) for i in range(2)]
    G = make_gpu_layer(L, pool, max_tokens=64, K=K)
    R = make_gpu_layer(L, pool, max_tokens=64, K=K)
    for i in range(2):
        out = run_layer(G, x[i], gpu)
        a = _decode_state(G, T, K, E, shared)
        R.route(T, x=to_dev(x[i], gpu))
        xq = G.read("xq", (T, 2048), np.int8)
        xs = G.read("xs", (T, 16), np.float32)
        xsum = G.read("xsum", (T, 16), np.int32)
        ref = R.experts(to_dev(xq, gpu), to_dev(xs, gpu), to_dev(xsum, gpu))
        torch.cuda.synchronize()
        r = _decode_state(R, T, K, E, shared)
        for name in r:
            assert np.array_equal(a[name].view(np.uint8), r[name].view(np.uint8)), f"forward {i}: {name} differs"
        assert np.array_equal(out.view(np.uint32), ref.cpu().numpy().view(np.uint32)), f"forward {i}: out differs"
        G.time_stage("gate_up", 2)
        assert np.array_equal(G.read("Z", a["Z"].shape, np.uint16), a["Z"]), "gate_up re-launch differs"
    G.close()
    R.close()


def test_decode_forward_plans_like_dispatch_random(gpu):
    """The self-planning decode forward against route + experts on 24 seeded draws of the shape (E, top-K, T from 1
    to 32, pool or not, shared expert or not, code mix): every buffer, the gate_up unit list and the output bit for
    bit, on one layer object per shape and three consecutive forwards (the routing masks are cleared in between)."""
    import torch
    rng = np.random.default_rng(2024)
    for case in range(24):
        E = int(rng.choice([64, 128, 256]))
        K = int(rng.integers(2, 9))
        T = int(rng.integers(1, 33))
        pool = int(rng.choice([E, 48, 16])) if E > 48 else E
        shared = bool(rng.integers(0, 2))
        mix = ["mixed", 2, 3, 4, 8][int(rng.integers(0, 5))]
        say(f"[decode plan random {case}] E={E} K={K} T={T} pool={pool} shared={shared} mix={mix}")
        # one matrix per code width, the other experts aliasing it: every expert keeps its width (the plan's classes)
        L = synth.make_layer(5000 + case, E=E, mix=mix, shared=shared, experts=[0])
        G = make_gpu_layer(L, pool, max_tokens=32, K=K)
        R = make_gpu_layer(L, pool, max_tokens=32, K=K)
        for i in range(3):
            x = synth.make_x(6000 + 10 * case + i, T)
            out = run_layer(G, x, gpu)
            a = _decode_state(G, T, K, E, shared)
            R.route(T, x=to_dev(x, gpu))
            ref = R.experts(to_dev(G.read("xq", (T, 2048), np.int8), gpu), to_dev(G.read("xs", (T, 16), np.float32), gpu),
                            to_dev(G.read("xsum", (T, 16), np.int32), gpu))
            torch.cuda.synchronize()
            r = _decode_state(R, T, K, E, shared)
            for name in r:
                assert np.array_equal(a[name].view(np.uint8), r[name].view(np.uint8)), f"case {case} forward {i}: {name}"
            assert np.array_equal(out.view(np.uint32), ref.cpu().numpy().view(np.uint32)), f"case {case} forward {i}: out"
        G.close()
        R.close()


@pytest.mark.parametrize("kind,T,pool", [
    ("zipf", 128, 256), ("skewed", 128, 256),
    ("zipf", 32, 256),    # one routing block: the decode kernels
    ("zipf", 32, 48),     # one routing block with the pool (scores first)
    ("skewed", 200, 48),  # several blocks with the pool
])
def test_logits_routing(gpu, kind, T, pool):
    """Routing from given logits; the A8 of x is written by the first per-token routing kernel."""
    say(f"[logits routing] {kind} T={T} pool={pool}")
    L = synth.make_layer(21, mix="mixed", shared=True, zero_bias=True)
    lg = synth.logits_zipf(5, T) if kind == "zipf" else synth.logits_skewed(5, T)
    G = make_gpu_layer(L, pool)
    x = synth.make_x(77, T)
    out = run_layer(G, x, gpu, logits=lg)
    r = oracle.Layer(L).forward(x, logits=lg, C=pool)
    assert np.array_equal(G.read("xq", (T, 2048), np.int8), r["xq"]), "A8 codes of x differ"
    assert np.array_equal(G.read("xs", (T, 16), np.float32).view(np.uint32), r["xs"].view(np.uint32))
    assert np.array_equal(G.read("xsum", (T, 16), np.int32), r["xsum"])
    check_full(G, r, T, 8, True)
    assert np.array_equal(out.view(np.uint32), r["out"].view(np.uint32))
    G.close()


@pytest.mark.parametrize("T,mix,kind", [
    (512, "mixed", "skewed"),    # 16 hot experts take half the slots: multi-chunk tiled units at every width
    (300, 8, "skewed"),          # 8-bit tiled units (zero term on the MFMA accumulator), ragged chunks
    (256, 2, "zipf"),
    (384, 4, "zipf"),
])
def test_tiled_units_bit_exact(gpu, T, mix, kind):
    """Experts with more than TILED_MIN slots run the tiled GEMM; every stage bit-exact against the oracle."""
    say(f"[tiled] T={T} mix={mix} {kind}")
    L = layer_for(mix, True, seed=61)
    lg = synth.logits_zipf(T + 1, T) if kind == "zipf" else synth.logits_skewed(T + 1, T)
    G = make_gpu_layer(L, 256, max_tokens=T)
    # (outlier channels only with the 2/3/4-bit mix: random 8-bit codes around random zeros would overflow fp16 Z)
    x = synth.make_x(500 + T, T, outlier_frac=0.01 if mix == "mixed" else 0.0)
    out = run_layer(G, x, gpu, logits=lg)
    assert np.isfinite(r_z := G.read("Z", (T * 9, 512), np.uint16).view(np.float16)).all(), "Z overflowed fp16"
    r = oracle.Layer(L).forward(x, logits=lg, C=256)
    assert (r["count"] > 40).sum() >= 8, "the case must exercise tiled units"
    check_full(G, r, T, 8, True)
    assert np.array_equal(out.view(np.uint32), r["out"].view(np.uint32)), "combine not bit-exact"
    G.close()


def test_tiled_absent_token_stores_dropped(gpu):
    """The tiled gate_up issues its Z stores (2/3/4-bit codes) from every lane and relies on the buffer range check
    to drop those of absent tokens (rows slot0 + n, n >= ntok, of a chunk). All-2-bit layer without the shared
    expert, T = 100, logits that put every token on the last expert: its 100 slots are the last of the layer, split
    into tiled chunks, so a store of an absent token that was not dropped would land in the rows past the last
    slot. Those rows of the workspace, filled with a sentinel first, must keep it; Z and the output stay
    bit-exact."""
    import ctypes
    T, Tmax, E = 100, 160, 256
    say(f"[tiled stores] T={T} max_tokens={Tmax}")
    L = layer_for(2, False, seed=62)
    lg = synth.logits_zipf(T + 3, T)
    lg[:, E - 1] += 100.0                      # every token's first choice
    G = make_gpu_layer(L, 256, max_tokens=Tmax)
    rows = Tmax * 9
    sentinel = np.full((rows, 512), 0x7E7E, np.uint16)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(G.buffers().Z, sentinel.ctypes.data, sentinel.nbytes, 1) == 0   # host to device
    x = synth.make_x(700, T)
    out = run_layer(G, x, gpu, logits=lg)
    S = T * 8
    Z = G.read("Z", (rows, 512), np.uint16)
    r = oracle.Layer(L).forward(x, logits=lg, C=256)
    assert r["count"][E - 1] == T, "every token must pick the last expert"
    assert (Z[S:] == 0x7E7E).all(), "a store of an absent token reached the rows past the last slot"
    assert np.array_equal(Z[:S], r["Z"]), "Z not bit-exact"
    assert np.array_equal(out.view(np.uint32), r["out"].view(np.uint32)), "combine not bit-exact"
    G.close()


@pytest.mark.parametrize("T,mix,shared,pool,kind", [
    (512, "mixed", True, 48, None),       # config 2: router x Wr with outlier channels, block pool 48
    (2048, "mixed", True, 256, "zipf"),   # one layer of config 3
    (4096, 2, False, 256, "uniform"),     # config 4, 2-bit
    (4096, 2, False, 256, "skewed"),      # config 4, 2-bit, 16 experts take half the slots
    (4096, 4, False, 256, "uniform"),     # config 4, 4-bit
    (4096, 4, False, 256, "skewed"),
    (4096, 8, False, 256, "uniform"),     # config 4, 8-bit (W8A8)
    (4096, 8, False, 256, "skewed"),
    (5120, 4, False, 256, "uniform"),     # 160 routing blocks: more block masks than the planner holds in registers
])
def test_full_size_batch_invariance(gpu, T, mix, shared, pool, kind):
    """At the configs' full token counts the GPU layer runs every expert through the work lists and chunking of
    that size; a token's output depends only on its own routing block, so the rows of a few whole 32-token
    blocks must equal, bit for bit, the oracle run on those blocks alone (indices, weights and outputs)."""
    say(f"[full size] T={T} mix={mix} shared={shared} pool={pool} {kind}")
    L = synth.make_layer(7 + T, mix=mix, shared=shared, zero_bias=kind is not None, w8_symmetric=False)
    x = synth.make_x(900 + T, T, outlier_frac=0.01 if mix == "mixed" else 0.0)
    lg = None
    if kind == "zipf":
        lg = synth.logits_zipf(T + 3, T)
    elif kind == "skewed":
        lg = synth.logits_skewed(T + 3, T)
    elif kind == "uniform":
        lg = np.random.default_rng(T + 3).standard_normal((T, 256)).astype(np.float32)
    G = make_gpu_layer(L, pool, max_tokens=T)
    out = run_layer(G, x, gpu, logits=lg)
    topk = G.read("topk", (T, 8), np.int32)
    topw = G.read("topw", (T, 8), np.float32)
    count = G.read("count", (256,), np.int32)   # routed slots per expert
    G.close()
    assert count.sum() == 8 * T
    if T >= 2048:
        assert (count > 64).sum() >= 8, "the case must run multi-chunk tiled experts"
    nb = T // 32
    blocks = [0, nb // 3, nb - 1]
    rows = np.concatenate([np.arange(32 * b, 32 * b + 32) for b in blocks])
    r = oracle.Layer(L).forward(x[rows], logits=None if lg is None else lg[rows], C=pool)
    assert np.array_equal(topk[rows], r["topk"]), "expert indices differ"
    assert np.array_equal(topw[rows].view(np.uint32), r["topw"].view(np.uint32)), "routing weights differ"
    close(out[rows], r["out"], "out")
    assert np.array_equal(out[rows].view(np.uint32), r["out"].view(np.uint32)), "output rows not bit-exact"


@pytest.mark.parametrize("T,pool", [(32, 256), (32, 48), (200, 48)])
def test_experts_norm_bit_exact(gpu, T, pool):
    """llmoe_experts_norm: combine + FWHT-2048 un-rotation + residual + next-layer RMSNorm / rotation / A8."""
    import torch
    say(f"[experts_norm] T={T} pool={pool}")
    L = layer_for("mixed", True)
    G = make_gpu_layer(L, pool)
    x = synth.make_x(900 + T, T)
    signs = np.where(np.random.default_rng(T).random(2048) < 0.5, -1.0, 1.0).astype(np.float32)
    h0 = (np.random.default_rng(T + 1).standard_normal((T, 2048)) * 2).astype(np.float32)
    xq, xs, xsum = oracle.quant_a8(x)
    dx = [to_dev(a, gpu) for a in (xq, xs, xsum)]
    G.route(T, x=to_dev(x, gpu))
    h = to_dev(h0, gpu)
    q, s, sm = G.experts_norm(*dx, to_dev(signs, gpu), 1e-6, h)
    torch.cuda.synchronize()
    r = oracle.Layer(L).forward(x, C=pool)
    hn, rq, rs, rsm = oracle.combine_norm(r["Y"], r["tok_slots"], 9, signs, 1e-6, h0)
    assert np.array_equal(h.cpu().numpy().view(np.uint32), hn.view(np.uint32)), "residual not bit-exact"
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(sm.cpu().numpy(), rsm)
    G.close()


@pytest.mark.parametrize("T,pool,logits", [(32, 256, False), (32, 48, False), (5, 256, True), (200, 48, False)])
def test_forward_norm_matches_route_experts_norm(gpu, T, pool, logits):
    """llmoe_layer_forward_norm (at decode the self-planning gate_up) against llmoe_route + llmoe_experts_norm on the
    same layer and inputs: h, q_next, s_next and sum_next bit for bit, on two consecutive calls."""
    import torch
    say(f"[forward_norm] T={T} pool={pool} logits={logits}")
    L = layer_for("mixed", True)
    G = make_gpu_layer(L, pool)
    signs = to_dev(np.where(np.random.default_rng(5).random(2048) < 0.5, -1.0, 1.0).astype(np.float32), gpu)
    for i in range(2):
        x = to_dev(synth.make_x(3000 + 10 * T + i, T), gpu)
        lg = to_dev(synth.logits_zipf(3100 + i, T), gpu) if logits else None
        h0 = torch.randn((T, 2048), device=gpu)
        h1 = h0.clone()
        a = G.forward_norm(x, signs, 1e-6, h1, logits=lg)
        torch.cuda.synchronize()
        a = [t.clone() for t in a]
        h2 = h0.clone()
        if logits:
            G.route(T, logits=lg)
            xq, xs, xsum = (to_dev(v, gpu) for v in oracle.quant_a8(x.cpu().numpy()))
        else:
            G.route(T, x=x)
            xq, xs, xsum = G.read("xq", (T, 2048), np.int8), G.read("xs", (T, 16), np.float32), G.read("xsum", (T, 16), np.int32)
            xq, xs, xsum = to_dev(xq, gpu), to_dev(xs, gpu), to_dev(xsum, gpu)
        b = G.experts_norm(xq, xs, xsum, signs, 1e-6, h2)
        torch.cuda.synchronize()
        assert torch.equal(h1.view(torch.int32), h2.view(torch.int32)), f"call {i}: h differs"
        for name, u, v in zip(("q_next", "s_next", "sum_next"), a, b):
            assert torch.equal(u.view(torch.uint8), v.view(torch.uint8)), f"call {i}: {name} differs"
    G.close()


def test_layer_load_matches_create(gpu, tmp_path):
    """llmoe_layer_load from a model directory in the reference's format == llmoe_layer_create on the same data."""
    say("[load] model dir")
    L = layer_for("mixed", True)
    ref = synth.write_model_dir(tmp_path, L, li=3)
    Gl = Layer.load(tmp_path, 3, max_tokens=64)
    Gc = Layer(ref["blob"], ref["gu_off"], ref["d_off"], ref["bits"], ref["bias"], ref["Wr"], n_experts=256, top_k=8,
               pool=48, has_shared=True, max_tokens=64)
    x = synth.make_x(21, 32)
    a = run_layer(Gl, x, gpu)
    b = run_layer(Gc, x, gpu)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    r = oracle.Layer(ref).forward(x, C=48)
    assert np.array_equal(a.view(np.uint32), r["out"].view(np.uint32))
    Gl.close()
    Gc.close()


@pytest.mark.parametrize("T,bits,R", [(1, 8, 3072), (16, 4, 512), (32, 2, 1024), (32, 3, 512), (100, 8, 512),
                                      (300, 4, 768), (77, 2, 256)])
def test_dense_bit_exact(gpu, T, bits, R):
    """llmoe_dense_forward (streamed for T <= 32, tiled above) == orc_dense, store and accumulate."""
    import torch
    from llmoe import Dense
    say(f"[dense] T={T} bits={bits} R={R}")
    c, s_, z = gen.matrix(4000 + bits + R, R, 2048, bits)
    blob = oracle.pack_i8(c, s_, z, bits)
    x = synth.make_x(4100 + T, T)
    xq, xs, xsum = oracle.quant_a8(x)
    D = Dense(blob, R, bits, max_tokens=512)
    dx = [to_dev(a, gpu) for a in (xq, xs, xsum)]
    y = D.forward(*dx)
    torch.cuda.synchronize()
    ref = oracle.dense(blob, R, 2048, bits, xq, xs, xsum)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32)), "dense not bit-exact"
    y0 = np.random.default_rng(T).standard_normal((T, R)).astype(np.float32)
    yd = to_dev(y0, gpu)
    D.forward(*dx, out=yd, accumulate=True)
    torch.cuda.synchronize()
    ref2 = oracle.dense(blob, R, 2048, bits, xq, xs, xsum, y=y0)
    assert np.array_equal(yd.cpu().numpy().view(np.uint32), ref2.view(np.uint32)), "dense accumulate not bit-exact"
    D.close()


def test_router_logits_bit_exact(gpu):
    T = 70
    say(f"[router logits] T={T}")
    L = layer_for("mixed", True)
    G = make_gpu_layer(L, 256)
    x = synth.make_x(3, T)
    run_layer(G, x, gpu)
    part = G.read("logits_part", (8, T, 256), np.float32)
    lg = part[0].copy()
    for c in range(1, 8):
        lg = (lg + part[c]).astype(np.float32)
    ref = oracle.router_logits(x, L["Wr"])
    assert np.array_equal(lg.view(np.uint32), ref.view(np.uint32))
    G.close()


def test_external_dispatch(gpu):
    """llmoe_dispatch + llmoe_experts with externally given routing (uniform random distinct experts)."""
    import torch
    T, K = 64, 8
    say(f"[dispatch] T={T}")
    L = layer_for("mixed", True)
    G = make_gpu_layer(L, 256)
    rng = np.random.default_rng(9)
    topk = np.stack([rng.choice(256, K, replace=False) for _ in range(T)]).astype(np.int32)
    topw = rng.uniform(0.05, 0.6, (T, K)).astype(np.float32)
    x = synth.make_x(4, T)
    xq, xs, xsum = oracle.quant_a8(x)
    G.dispatch(to_dev(topk, gpu), to_dev(topw, gpu))
    out = G.experts(to_dev(xq, gpu), to_dev(xs, gpu), to_dev(xsum, gpu))
    torch.cuda.synchronize()
    r = oracle.Layer(L).experts(xq, xs, xsum, topk, topw)
    r.update(topk=topk, topw=topw)
    check_full(G, r, T, K, True)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), r["out"].view(np.uint32))
    G.close()


@pytest.mark.parametrize("T,pool", [(32, 256), (32, 48), (200, 48)])
def test_hip_graph_replays(gpu, T, pool):
    """The layer forward and a dense projection captured in one HIP graph: every replay, with eager calls on other
    inputs and host synchronisations in between, reproduces the eager results bit for bit (the calls allocate,
    clear and synchronise nothing, and keep no host state between launches)."""
    import torch
    from llmoe import Dense
    say(f"[graph] T={T} pool={pool}")
    L = layer_for("mixed", True)
    G = make_gpu_layer(L, pool)
    R = 1024
    c, s_, z = gen.matrix(4500, R, 2048, 8)
    D = Dense(oracle.pack_i8(c, s_, z, 8), R, 8, max_tokens=256)
    x = to_dev(synth.make_x(60 + T, T), gpu)
    x2 = to_dev(synth.make_x(61 + T, T), gpu)
    xq, xs, xsum = (to_dev(a, gpu) for a in oracle.quant_a8(synth.make_x(62 + T, T)))
    out = torch.empty((T, 2048), dtype=torch.float32, device=gpu)
    y = torch.empty((T, R), dtype=torch.float32, device=gpu)
    G.forward(x, out=out)
    D.forward(xq, xs, xsum, out=y)
    torch.cuda.synchronize()
    ref_out, ref_y = out.clone(), y.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        G.forward(x, out=out)
        D.forward(xq, xs, xsum, out=y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        G.forward(x, out=out)
        D.forward(xq, xs, xsum, out=y)
    for i in range(4):
        out.zero_()
        y.zero_()
        other = G.forward(x2)                  # eager work on the same layer object between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref_out.view(torch.int32)), f"replay {i}: layer output differs"
        assert torch.equal(y.view(torch.int32), ref_y.view(torch.int32)), f"replay {i}: dense output differs"
        assert not torch.equal(other, ref_out)
    del g
    D.close()
    G.close()
