#!/usr/bin/env python3
"""Benchmark of the LLaDA2 routed-expert MoE layer on one MI355X through libllmoe.so.

Headline workload (value): config 1 -- one MoE layer, 32 tokens (one denoising block), hidden 2048, 256
routed experts at the shipped 2/3/4-bit mix (61/34/6 %), uniform-random top-8 of sigmoid(x Wr), plus the W8A8
shared expert; a step is one full layer pass (A8 of x -> router -> routing -> gate_up (which also builds the slot
plan) -> FWHT-512 + A8 -> down -> combine) with x already resident in HBM. Also measured (fields "configs"): config 0 (32 tokens, all
4-bit, block pool 48, no shared expert), config 2 (512 tokens), config 3 (2048 tokens through a stack of 20
independently seeded layers with Zipf(1.1) expert load), config 4 (4096 tokens at 2/4/8 bits, uniform and skewed
routing) and the dense projection at 32 and 2048 tokens.

Roofline: the dominant kernel is the gate_up expert GEMM (two thirds of the weight bytes; at decode the kernel that
also plans the slots from the routing masks); its algorithmic bytes per launch are the packed gate_up bytes of every
expert the step touches (each streamed exactly once) plus the shared expert's, and its duration is measured with
HIP events on the launch stream (re-launches of the step's own gate_up kernel, llmoe_layers_time_stage).

CPU baseline: the CPU oracle (oracle/, the C restatement of the reference's path, OpenMP over experts) timed on
the host cores on the same config-1 layer and input, repeated for a bounded ~10 s.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "llada2-orin-cuda_amd"), str(ROOT / "oracle")]

import numpy as np  # noqa: E402

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0        # MI355X dense int8 MFMA (TOP/s)
H, I, K, E = 2048, 512, 8, 256


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_gpu_layer(llmoe, L, pool, max_tokens):
    return llmoe.Layer(L["blob"], L["gu_off"], L["d_off"], L["bits"], L["bias"], L["Wr"], n_experts=E, top_k=K,
                       pool=pool, has_shared=L["shared"], max_tokens=max_tokens)


def gate_up_bytes(L, topk):
    from llmoe import synth
    used = np.unique(topk.reshape(-1))
    b = sum(synth.matrix_bytes(2 * I, H, int(L["bits"][e])) for e in used)
    if L["shared"]:
        b += synth.matrix_bytes(2 * I, H, 8)
    return int(b)


def down_bytes(L, topk):
    from llmoe import synth
    used = np.unique(topk.reshape(-1))
    b = sum(synth.matrix_bytes(H, I, int(L["bits"][e])) for e in used)
    if L["shared"]:
        b += synth.matrix_bytes(H, I, 8)
    return int(b)


def time_steps(fn, steps, warmup):
    """fn(i) runs step i; W untimed warmup steps, then exactly `steps` timed steps between synchronisations."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def stage_profile(G, fn, reps=20):
    import torch
    G.set_profiling(True)
    acc = {}
    for i in range(reps):
        fn(i)
        for k, v in G.stage_ms().items():
            acc.setdefault(k, []).append(v)
    G.set_profiling(False)
    torch.cuda.synchronize()
    return {k: float(np.median(v)) for k, v in acc.items()}


def decode_layers(llmoe, synth, torch, seed, T, mix, shared, pool, nlayers=4, zero_bias=False):
    """The layers, input and step function of a decode configuration. A step is one layer pass; consecutive steps
    cycle through `nlayers` independently seeded layers so the weights (> 256 MB in total) stream from HBM, not from
    the last-level cache. zero_bias: the router runs with a zero expert bias, so the experts are exchangeable and
    each token's top-8 is a uniformly random 8-subset."""
    dev = torch.device("cuda:0")
    Ls = [synth.make_layer(seed + 1000 * i, mix=mix, shared=shared, zero_bias=zero_bias) for i in range(nlayers)]
    Gs = [make_gpu_layer(llmoe, L, pool, T) for L in Ls]
    x = torch.from_numpy(synth.make_x(seed + 1, T)).to(dev)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)
    fn = lambda i: Gs[i % nlayers].forward(x, out=out)  # noqa: E731
    return {"Ls": Ls, "Gs": Gs, "x": x, "out": out, "fn": fn, "T": T, "shared": shared}


def decode_timing(d, steps, warmup):
    """The contract's timing of a decode configuration: W warm-up steps, then exactly `steps` timed steps. With short
    arguments (fewer than 200 steps or 300 warm-up steps) the same steps are re-timed after 300 more warm-up steps
    and reported beside it as `steady_state` (the contract's figure stays the first): a GPU that has been idle
    clocks down, and 20-step windows then go from about 0.059 to 0.0555 ms per config-1 step over ~10 ms of work."""
    dt = time_steps(d["fn"], steps, warmup)
    steady = None
    if steps < 200 or warmup < 300:
        steady = {"steps": 200, "warmup": 300, "ms_per_step": time_steps(d["fn"], 200, 300) / 200 * 1e3}
    return dt, steady


def one_layer_config(llmoe, synth, torch, name, seed, T, mix, shared, pool, steps, warmup, nlayers=4,
                     zero_bias=False, layers=None, timing=None):
    """A decode configuration's bench entry. layers / timing: from decode_layers / decode_timing when the caller
    builds and times the configuration itself."""
    d = layers or decode_layers(llmoe, synth, torch, seed, T, mix, shared, pool, nlayers, zero_bias)
    Ls, Gs, x, out, fn = d["Ls"], d["Gs"], d["x"], d["out"], d["fn"]
    nlayers = len(Gs)
    dt, steady = timing or decode_timing(d, steps, warmup)
    prof = stage_profile(Gs[0], lambda i: Gs[0].forward(x, out=out))
    for G in Gs:
        G.forward(x, out=out)
    # steady-state kernel durations: back-to-back launches cycling through the layers, between two HIP events on
    # the launch stream
    prof["gate_up"] = llmoe.time_stage_layers(Gs, "gate_up", 20)
    prof["down"] = llmoe.time_stage_layers(Gs, "down", 20)
    topks = [G.read("topk", (T, K), np.int32) for G in Gs]
    gub = float(np.mean([gate_up_bytes(L, t) for L, t in zip(Ls, topks)]))
    dnb = float(np.mean([down_bytes(L, t) for L, t in zip(Ls, topks)]))
    slots = T * K + (T if shared else 0)
    t_w = (prof["gate_up"] + prof["down"]) * 1e-3
    res = {
        "workload": name, "tokens": T, "layers_cycled": nlayers, "ms_per_step": dt / steps * 1e3,
        "tokens_per_s": T * steps / dt, "experts_touched": float(np.mean([np.unique(t).size for t in topks])),
        "weight_bytes": gub + dnb, "weight_stream_GBps": (gub + dnb) / t_w / 1e9,
        "weight_stream_frac_peak": (gub + dnb) / t_w / 1e9 / PEAK_HBM_GBS,
        "int8_TOPS": 2 * slots * 3 * I * H / t_w / 1e12,
        "stage_ms": prof, "gate_up_bytes": gub, "down_bytes": dnb,
    }
    if steady:
        res["steady_state"] = steady
    res["fast_numerics"] = fast_numerics(llmoe, Gs, fn, steps, warmup, T)
    for G in Gs:
        G.forward(x, out=out)
    return res, (Ls[0], Gs, x, out, fn)


def norm_step(llmoe, torch, Gs, x, steps, warmup):
    """The layer step with the fused combine epilogue (llmoe_layer_forward_norm): routing, experts, combine + FWHT-2048
    un-rotation + residual add + the next layer's RMSNorm / rotation / A8, cycling through the same layers."""
    T = x.shape[0]
    dev = x.device
    signs = torch.from_numpy(np.where(np.random.default_rng(5).random(H) < 0.5, -1.0, 1.0).astype(np.float32)).to(dev)
    h = torch.randn((T, H), device=dev)
    nxt = (torch.empty((T, H), dtype=torch.int8, device=dev), torch.empty((T, 16), dtype=torch.float32, device=dev),
           torch.empty((T, 16), dtype=torch.int32, device=dev))

    def fn(i):
        Gs[i % len(Gs)].forward_norm(x, signs, 1e-6, h, out=nxt)

    dt = time_steps(fn, steps, warmup)
    comb = llmoe.time_stage_layers(Gs, "combine", 20)
    for G in Gs:   # leave each layer's latest call a plain forward again
        G.forward(x)
    return {"ms_per_step": dt / steps * 1e3, "tokens_per_s": T * steps / dt, "combine_norm_ms": comb,
            "combine_ms": llmoe.time_stage_layers(Gs, "combine", 20)}


FAST = True   # measure each configuration in LLMOE_NUMERICS_FAST as well (--no-fast: exact mode only)


def fast_numerics(llmoe, Gs, fn, steps, warmup, tokens, layers_per_step=1):
    """The same step with LLMOE_NUMERICS_FAST (the gate_up SiLU by the hardware transcendentals; fp16 slot outputs
    for several routing blocks): step time and the steady-state gate_up duration; the layers are left in exact
    mode. None when FAST is off."""
    if not FAST:
        return None
    for G in Gs:
        G.set_numerics(True)
    dt = time_steps(fn, steps, warmup)
    gu = llmoe.time_stage_layers(Gs, "gate_up", 5)
    for G in Gs:
        G.set_numerics(False)
    return {"ms_per_step": dt / steps * 1e3, "tokens_per_s": tokens * steps / dt, "gate_up_ms": gu}


def spot_check(L, out_rows, x_rows, lg_rows, pool):
    """One routing block of a timed configuration against the CPU oracle, outside the timed region: the block's
    routing depends on its own tokens only, so the oracle runs on those rows alone."""
    import oracle
    r = oracle.Layer(L).forward(np.ascontiguousarray(x_rows), logits=None if lg_rows is None else
                                np.ascontiguousarray(lg_rows), C=pool)
    err = float(np.abs(out_rows - r["out"]).max()) / max(float(np.abs(r["out"]).max()), 1e-30)
    exact = bool(np.array_equal(out_rows.view(np.uint32), r["out"].view(np.uint32)))
    if not exact:
        log(f"[bench] WARNING: spot check differs from the oracle (max rel err {err:.3e})")
    return {"rows": f"0-{out_rows.shape[0] - 1}", "bit_exact": exact, "max_abs_err_rel": err}


def stack_config(llmoe, synth, torch, steps, warmup, nlayers=20, T=2048):
    """Config 3: 2048 tokens through 20 independently seeded mixed-bit layers (+ shared), Zipf(1.1) load."""
    dev = torch.device("cuda:0")
    layers, logits = [], []
    wbytes = 0
    t0 = time.perf_counter()
    for li in range(nlayers):
        L = synth.make_layer(1000 + li, mix="mixed", shared=True, zero_bias=True)
        layers.append((L, make_gpu_layer(llmoe, L, 256, T)))
        logits.append(torch.from_numpy(synth.logits_zipf(2000 + li, T)).to(dev))
        if li:
            del L["blob"]
    log(f"[bench] config 3: {nlayers} layers built in {time.perf_counter() - t0:.1f} s")
    x_np = synth.make_x(7, T)
    x = torch.from_numpy(x_np).to(dev)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)

    def fn(i):
        for (L, G), lg in zip(layers, logits):
            G.forward(x, lg, out=out)

    dt = time_steps(fn, steps, warmup)
    # per-layer stage profile and weight bytes
    for (L, G), lg in zip(layers, logits):
        G.forward(x, lg, out=out)
        topk = G.read("topk", (T, K), np.int32)
        wbytes += gate_up_bytes(L, topk) + down_bytes(L, topk)
    Gs = [G for _, G in layers]
    L0, G0 = layers[0]
    G0.forward(x, logits[0], out=out)
    torch.cuda.synchronize()
    check = spot_check(L0, out[:32].cpu().numpy(), x_np[:32], logits[0][:32].cpu().numpy(), 256)
    gu = llmoe.time_stage_layers(Gs, "gate_up", 3)
    dn = llmoe.time_stage_layers(Gs, "down", 3)
    gu_ms, dn_ms = [gu] * nlayers, [dn] * nlayers
    fast = fast_numerics(llmoe, Gs, fn, steps, warmup, T)
    t_w = (sum(gu_ms) + sum(dn_ms)) * 1e-3
    slots = T * (K + 1) * nlayers
    res = {
        "workload": "config 3: 2048 tokens x 20 layers, mixed 2/3/4-bit + W8A8 shared, Zipf(1.1) load",
        "tokens": T, "layers": nlayers, "ms_per_step": dt / steps * 1e3,
        "tokens_per_s_per_layer": T * nlayers * steps / dt, "stack_tokens_per_s": T * steps / dt,
        "weight_bytes": wbytes, "weight_stream_GBps": wbytes / t_w / 1e9,
        "weight_stream_frac_peak": wbytes / t_w / 1e9 / PEAK_HBM_GBS,
        "int8_TOPS": 2 * slots * 3 * I * H / t_w / 1e12,
        "int8_mfma_frac_peak": 2 * slots * 3 * I * H / t_w / 1e12 / PEAK_INT8_TOPS,
        "gate_up_ms_per_layer": float(np.mean(gu_ms)), "down_ms_per_layer": float(np.mean(dn_ms)),
        "spot_check_layer0": check, "fast_numerics": fast,
    }
    for _, G in layers:
        G.close()
    return res


TRAFFIC_FILE = ROOT / "profiles" / "expert_gemm_gate_up_config1_traffic.txt"


def measured_traffic():
    """HBM bytes per gate_up launch from the committed rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE per
    dispatch, calibrated against a copy kernel of known size); None when no such summary exists."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split("=")[1].split()[0])
    return None


PROFILE_3_TRAFFIC = ROOT / "profiles" / "tiled_gemm_config3_traffic.txt"
PROFILE_3_STATS = ROOT / "profiles" / "tiled_gemm_config3_kernel_stats.txt"


def profile_column(path, kernel, col):
    """Column `col` (0 = the kernel name) of the row for `kernel` in a committed rocprofv3 summary table, or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        f = line.split()
        if f and f[0] == kernel and len(f) > col:
            try:
                return float(f[col])
            except ValueError:
                return None
    return None


def roofline_2048(c3):
    """Weight-stream roofline of one config-3 layer (2048 tokens): the tiled gate_up + down GEMMs' algorithmic
    weight bytes over their steady-state durations (HIP events on the launch stream, the 20 layers launched in
    turn), the int8 MFMA rate of the same phase, and the HBM bytes the committed rocprofv3 summaries measured for the
    two kernels (calibrated FETCH_SIZE + WRITE_SIZE per launch) against the algorithmic bytes."""
    per_layer = c3["weight_bytes"] / c3["layers"]
    t = (c3["gate_up_ms_per_layer"] + c3["down_ms_per_layer"]) * 1e-3
    ops = 2 * c3["tokens"] * (K + 1) * 3 * I * H
    gu_mb = profile_column(PROFILE_3_TRAFFIC, "tiled_gemm<0>", 4)
    dn_mb = profile_column(PROFILE_3_TRAFFIC, "tiled_gemm<1>", 4)
    traffic = None if gu_mb is None or dn_mb is None else (gu_mb + dn_mb) * 1e6
    # algorithmic bytes of the two launches: weights, the gathered A8 rows of x (2 KB + 128 B per slot), Z written
    # and Z' read (1 KB + 512 B and 512 B + 32 B per slot), Y written (8 KB per slot)
    slots = c3["tokens"] * (K + 1)
    algo = per_layer + slots * (2048 + 128 + 1024 + 544 + 8192)
    gu_us = profile_column(PROFILE_3_STATS, "tiled_gemm<0>", 2)
    dn_us = profile_column(PROFILE_3_STATS, "tiled_gemm<1>", 2)
    achieved = per_layer / t / 1e9
    return {"bound": "hbm", "kernel": "tiled_gemm<gate_up> + tiled_gemm<down> (config 3, one 2048-token layer)",
            "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
            "weight_bytes_per_layer": per_layer, "gate_up_ms": c3["gate_up_ms_per_layer"],
            "down_ms": c3["down_ms_per_layer"], "int8_TOPS": ops / t / 1e12,
            "int8_mfma_frac": ops / t / 1e12 / PEAK_INT8_TOPS, "traffic": traffic,
            "algorithmic_bytes": algo, "traffic_ratio": None if traffic is None else traffic / algo,
            "rocprof_avg_us": {"gate_up": gu_us, "down": dn_us}}


def copy_calibration(torch, mib=512, reps=3):
    """Plain device copies of a known size, so counter runs can calibrate FETCH_SIZE / WRITE_SIZE per byte."""
    a = torch.empty(mib << 20, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    a.fill_(1)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"[bench] copy calibration: {reps} copies of {mib} MiB")


def prefill_config(llmoe, synth, torch, name, T, mix, shared, pool, logits_kind, steps, warmup, nlayers=2,
                   outliers=0.0):
    """One layer of T tokens (configs 2 and 4): a step is one full layer pass; the layers cycle so their weights
    stream from HBM. logits_kind: None (router x Wr), "uniform" (random logits), "skewed" (16 experts take half
    of the slots)."""
    dev = torch.device("cuda:0")
    Ls = [synth.make_layer(300 + 7 * i, mix=mix, shared=shared, zero_bias=logits_kind is not None)
          for i in range(nlayers)]
    Gs = [make_gpu_layer(llmoe, L, pool, T) for L in Ls]
    x_np = synth.make_x(31, T, outlier_frac=outliers)
    x = torch.from_numpy(x_np).to(dev)
    lgs = [None] * nlayers
    if logits_kind == "uniform":
        lgs = [torch.from_numpy(np.random.default_rng(40 + i).standard_normal((T, E)).astype(np.float32)).to(dev)
               for i in range(nlayers)]
    elif logits_kind == "skewed":
        lgs = [torch.from_numpy(synth.logits_skewed(40 + i, T)).to(dev) for i in range(nlayers)]
    out = torch.empty((T, H), dtype=torch.float32, device=dev)
    fn = lambda i: Gs[i % nlayers].forward(x, lgs[i % nlayers], out=out)  # noqa: E731
    dt = time_steps(fn, steps, warmup)
    fn(0)
    torch.cuda.synchronize()
    check = spot_check(Ls[0], out[:32].cpu().numpy(), x_np[:32], None if lgs[0] is None else lgs[0][:32].cpu().numpy(),
                       pool)
    for i in range(nlayers):
        fn(i)
    gu = llmoe.time_stage_layers(Gs, "gate_up", 5)
    dn = llmoe.time_stage_layers(Gs, "down", 5)
    topks = [G.read("topk", (T, K), np.int32) for G in Gs]
    fast = fast_numerics(llmoe, Gs, fn, steps, warmup, T)
    wb = float(np.mean([gate_up_bytes(L, t) + down_bytes(L, t) for L, t in zip(Ls, topks)]))
    slots = T * K + (T if shared else 0)
    t_w = (gu + dn) * 1e-3
    for G in Gs:
        G.close()
    return {"workload": name, "tokens": T, "ms_per_step": dt / steps * 1e3, "tokens_per_s": T * steps / dt,
            "gate_up_ms": gu, "down_ms": dn, "weight_bytes": wb, "weight_stream_GBps": wb / t_w / 1e9,
            "weight_stream_frac_peak": wb / t_w / 1e9 / PEAK_HBM_GBS,
            "int8_TOPS": 2 * slots * 3 * I * H / t_w / 1e12,
            "int8_mfma_frac_peak": 2 * slots * 3 * I * H / t_w / 1e12 / PEAK_INT8_TOPS, "layers_cycled": nlayers,
            "spot_check_layer0": check, "fast_numerics": fast}


def dense_config(llmoe, synth, torch, R, bits, T, steps, warmup, nmat=40):
    """Dense W.A8 projection (llmoe_dense_forward, the qkv shape of the reference engine: [3072, 2048]): a step is
    one projection of T tokens' A8 rows; the steps cycle through nmat matrices (> 256 MB) so the weights stream
    from HBM."""
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(77)
    Ds = [llmoe.Dense(synth.random_matrix(rng, R, H, bits), R, bits, max_tokens=T) for _ in range(nmat)]
    xq, xs, xsum = llmoe.quantize_a8(torch.from_numpy(synth.make_x(9, T)).to(dev))
    y = torch.empty((T, R), dtype=torch.float32, device=dev)
    dt = time_steps(lambda i: Ds[i % nmat].forward(xq, xs, xsum, out=y), steps, warmup)
    # GPU time per projection: one projection per matrix captured back to back in a HIP graph, replayed (a Python
    # call per projection costs more host time than a 32-token projection takes on the GPU)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for D in Ds:
            D.forward(xq, xs, xsum, out=y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for D in Ds:
            D.forward(xq, xs, xsum, out=y)
    reps = max(3, steps // nmat)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    t_gpu = (time.perf_counter() - t0) / (reps * nmat)
    del g
    for D in Ds:
        D.close()
    t = dt / steps
    wb = synth.matrix_bytes(R, H, bits)
    return {"workload": f"dense W{bits}A8 projection [{R} x {H}] (qkv shape), {T} tokens", "tokens": T,
            "ms_per_step": t * 1e3, "tokens_per_s": T / t, "weight_bytes": wb, "weight_stream_GBps": wb / t / 1e9,
            "weight_stream_frac_peak": wb / t / 1e9 / PEAK_HBM_GBS, "int8_TOPS": 2 * T * R * H / t / 1e12,
            "int8_mfma_frac_peak": 2 * T * R * H / t / 1e12 / PEAK_INT8_TOPS,
            "graph_replay": {"us_per_projection": t_gpu * 1e6, "weight_stream_GBps": wb / t_gpu / 1e9,
                             "weight_stream_frac_peak": wb / t_gpu / 1e9 / PEAK_HBM_GBS}}


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def cpu_baseline_2048(synth, seconds):
    """The CPU oracle on one config-3 layer (2048 tokens, mixed bits + shared, Zipf(1.1) logits): whole passes until
    `seconds` have elapsed (at least one)."""
    import oracle
    threads = cpu_threads()
    L = synth.make_layer(1000, mix="mixed", shared=True, zero_bias=True)
    x = synth.make_x(7, 2048)
    lg = synth.logits_zipf(2000, 2048)
    O = oracle.Layer(L)
    n, t0 = 0, time.perf_counter()
    while True:
        O.forward(x, logits=lg, C=256, nthreads=threads)
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": 2048 * n / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} full pass(es) of one config-3 layer (2048 tokens, Zipf(1.1) logits) through the C oracle, "
                      f"{dt:.1f} s"}


def cpu_baseline(L, x_np, pool, seconds):
    import oracle
    threads = cpu_threads()
    O = oracle.Layer(L)
    T = x_np.shape[0]
    n, t0 = 0, time.perf_counter()
    while True:
        O.forward(x_np, C=pool, nthreads=threads)
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": T * n / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} full passes of the config-1 layer ({T} tokens) through the C oracle "
                      f"(A8, fixed-order router, routing, integer W*A8 experts, FWHT-512, combine), {dt:.1f} s"}


def prefill_steps(args, config):
    """(timed steps, warm-up steps) of a prefill configuration: a share of --steps / --warmup with floors, so that
    the 2048- and 4096-token half of the metric is never timed from one or two steps (config 3 is a 20-layer stack
    of ~5 ms per step, config 4 one layer of ~0.4-0.6 ms, config 2 one layer of ~0.13 ms), nor right after the
    layers are built: the warm-up is at least ~15 ms of GPU work (the GPU takes ~10-15 ms of steady work to reach its
    steady step time)."""
    if config == 3:
        return max(5, args.steps // 20), max(3, args.warmup // 10)
    if config == 4:
        return max(10, args.steps // 20), max(40, args.warmup // 20)
    return max(20, args.steps // 5), max(100, args.warmup // 3)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--no-stack", action="store_true", help="skip config 3 (20-layer, 2048-token stack)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-headline", action="store_true", help="config 1 only (profiling runs)")
    ap.add_argument("--only-stack", action="store_true", help="config 3 only (profiling runs of the tiled GEMM)")
    ap.add_argument("--only", choices=["config0", "config2", "config4-2", "config4-4", "config4-8"],
                    help="one configuration only (config 0 or a prefill one), printed as its own JSON line "
                         "(profiling runs)")
    ap.add_argument("--copy-calibration", action="store_true", help="run 512 MiB device copies first (counter runs)")
    ap.add_argument("--no-fast", action="store_true", help="exact numerics only (profiling runs of one kernel variant)")
    args = ap.parse_args()
    global FAST
    FAST = not args.no_fast
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (expert parallelism is a design note "
              "only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import llmoe
    from llmoe import synth
    llmoe.load_library()
    torch.cuda.set_device(0)
    if args.copy_calibration:
        copy_calibration(torch)

    if args.only:
        if args.only == "config0":
            r, (_, G0s, _, _, _) = one_layer_config(llmoe, synth, torch, "config 0: 32 tokens, 4-bit, pool 48, "
                                                    "no shared", 11, 32, 4, False, 48, args.steps, args.warmup)
            for G in G0s:
                G.close()
        elif args.only == "config2":
            r = prefill_config(llmoe, synth, torch, "config 2", 512, "mixed", True, 48, None, *prefill_steps(args, 2),
                               nlayers=4, outliers=0.01)
        else:
            bits = int(args.only[-1])
            r = [prefill_config(llmoe, synth, torch, f"config 4: {bits}-bit {kind}", 4096, bits, False, 256, kind,
                                *prefill_steps(args, 4), nlayers=1 if bits == 8 else 2)
                 for kind in ("uniform", "skewed")]
        print(json.dumps(r))
        return
    if args.only_stack:
        print(json.dumps(stack_config(llmoe, synth, torch, *prefill_steps(args, 3))))
        return
    # The two decode configurations are built first and timed back to back, config 0 first: config 1's window then
    # follows GPU work instead of the idle time of the layers' host-side set-up (which leaves the GPU clocked down
    # for its first ~10 ms of work). Each keeps its own W warm-up steps and K timed steps; config 0's window is the
    # one that starts on an idle GPU.
    log("[bench] config 1 (headline) and config 0: layers")
    d1 = decode_layers(llmoe, synth, torch, 1, 32, "mixed", True, 256, zero_bias=True)
    d0 = None if args.only_headline else decode_layers(llmoe, synth, torch, 11, 32, 4, False, 48)
    t0 = None
    if d0:
        log("[bench] config 0: timing")
        t0 = decode_timing(d0, args.steps, args.warmup)
    log("[bench] config 1 (headline): timing")
    t1 = decode_timing(d1, args.steps, args.warmup)
    c1, (L1, G1s, x1, _, _) = one_layer_config(llmoe, synth, torch, "config 1: 32 tokens, mixed 2/3/4-bit + W8A8 "
                                              "shared, uniform-random routing (router x Wr with zero bias, no pool)",
                                              1, 32, "mixed", True, 256, args.steps, args.warmup, zero_bias=True,
                                              layers=d1, timing=t1)
    c1["with_combine_norm"] = norm_step(llmoe, torch, G1s, x1, args.steps, args.warmup)
    configs = [c1]
    c3 = None
    if d0:
        log("[bench] config 0")
        c0, (_, G0s, _, _, _) = one_layer_config(llmoe, synth, torch, "config 0: 32 tokens, 4-bit, pool 48, "
                                                 "no shared", 11, 32, 4, False, 48, args.steps, args.warmup,
                                                 layers=d0, timing=t0)
        for G in G0s:
            G.close()
        configs.insert(0, c0)
    if not args.no_stack and not args.only_headline:
        log("[bench] config 2")
        configs.append(prefill_config(llmoe, synth, torch, "config 2: 512 tokens, mixed 2/3/4-bit + W8A8 shared, "
                                      "router x Wr with 1% outlier channels x20, block pool 48", 512, "mixed", True,
                                      48, None, *prefill_steps(args, 2), nlayers=4, outliers=0.01))
        log("[bench] config 3")
        c3 = stack_config(llmoe, synth, torch, *prefill_steps(args, 3))
        configs.append(c3)
        for T in (32, 2048):
            log(f"[bench] dense projection, {T} tokens")
            # (warm-up: ~15 ms of calls, as for the prefill configurations)
            configs.append(dense_config(llmoe, synth, torch, 3072, 8, T, max(5, args.steps // 4),
                                        2000 if T <= 32 else 400))
        for bits in (2, 4, 8):
            for kind in ("uniform", "skewed"):
                log(f"[bench] config 4: {bits}-bit {kind}")
                configs.append(prefill_config(llmoe, synth, torch, f"config 4: 4096 tokens, all experts {bits}-bit, "
                                              f"{kind} routing, no shared expert", 4096, bits, False, 256, kind,
                                              *prefill_steps(args, 4), nlayers=1 if bits == 8 else 2))

    p = c1["stage_ms"]
    gu_s = p["gate_up"] * 1e-3
    achieved = c1["gate_up_bytes"] / gu_s / 1e9
    roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, "traffic": measured_traffic(),
                "kernel": "expert_gemm_plan (config 1: the decode gate_up GEMM, planning its units)", "bytes_per_launch": c1["gate_up_bytes"],
                "avg_launch_ms": p["gate_up"]}
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline")
        cpu = cpu_baseline(L1, x1.cpu().numpy(), 256, args.cpu_seconds)
        if not args.only_headline:
            log("[bench] cpu baseline, 2048 tokens")
            cpu["at_2048_tokens"] = cpu_baseline_2048(synth, args.cpu_seconds)
    for G in G1s:
        G.close()
    line = {
        "metric": "MoE-layer tokens/sec at 32 & 2048 tokens; weight-stream HBM GB/s as % peak",
        "value": c1["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": c1["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic (seeded random packed weights and activations of the config shapes)",
        "config": {"workload": c1["workload"], "tokens": 32, "hidden": H, "inter": I, "experts": E, "top_k": K,
                   "parallelism": "single GPU"},
        "weight_stream_GBps": c1["weight_stream_GBps"], "weight_stream_frac_peak": c1["weight_stream_frac_peak"],
        "roofline": roofline, "roofline_2048": roofline_2048(c3) if c3 else None, "cpu_baseline": cpu,
        "configs": configs,
    }
    if "steady_state" in c1:   # short arguments: the same steps re-timed after 300 more warm-up steps (not `value`)
        ss = c1["steady_state"]
        line["steady_state"] = dict(ss, tokens_per_s=32 / (ss["ms_per_step"] * 1e-3))
    print(json.dumps(line))


if __name__ == "__main__":
    main()
