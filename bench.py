#!/usr/bin/env python3
"""Benchmark of the small-M affine-quantised matmul on one MI355X.

Workload (the headline configuration): y[M,17408] = x[M,5120] . dequant(W)^T, W 4-bit
group 64 in MLX's affine layout, bf16 activations / scales / biases / output, M swept over
1..6, 8 (and 16).  A "step" is one call at M = 8 (a verify pass's width).

Method:
  * 8 distinct weight sets (~400 MB, more than the 256 MB Infinity Cache) are rotated so
    every call streams its weights from HBM: a graph holds whole cycles through every set
    (at least `steps` calls), so 350 MB of other weights pass between two uses of one set,
    also across the boundary between replays;
  * the calls of one M are captured into one HIP graph on a non-default stream and
    replayed R >= 10 times (at least 200 calls); HIP events on that stream bracket each
    replay, so a replay's time / calls is the back-to-back time per call including launch
    gaps; us_per_call is the median over the replays, with p10 / p90 beside it;
  * algorithmic bytes per call = N*K*bits/8 + 2*N*(K/gs)*2 + M*K*2 + M*N*2;
  * read_ceiling: the library's plain streaming-read kernel moving the M=8 call's
    algorithmic bytes per launch over the same rotation, timed the same way: the
    single-launch read rate this memory system reaches with no compute;
  * stock: the stock path a swapped layer falls through to (dfq_qmm_fallback, a GEMV) beside
    the fast kernel at 1..8 rows, and the fewest rows at which the fast kernel wins (the
    drop-in window's lower bound on this chip); at one row also for C1;
  * the CPU baseline is the oracle's fp32 restatement of MLX's CPU algorithm (dequantise a
    group, multiply-accumulate), OpenMP over the host cores, timed on a bounded sample: an
    MLX-semantics CPU restatement, not MLX;
  * the 64-layer verify forward (c5_chain*) is timed with one HIP graph per layer, launched
    one by one or composed into one launch, and as one captured graph; c5_rows times the
    composed fused forward at every verify width of the reference's --rows sweep.

--profile-timed dispatches the matmul only as graph replays (one warm-up replay, then the
timed ones), so that `rocprofv3 --kernel-trace --stats` averages the calls the figures time.

Prints ONE JSON line.  --gpus > 1 is refused: the benchmark measures one GPU.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "dflash-swift_amd"))

N_OUT, K_IN, BITS, GS = 17408, 5120, 4, 64
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20   # MI355X Infinity Cache: a weight set re-read sooner could hit it
# rocprofv3 summary of the M=8 launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated); the
# roofline's measured-traffic figure is read from its "traffic_bytes_per_launch:" line.
PROFILE = os.path.join(ROOT, "profiles", "qmm_mt8_b4g64_bf16_k5120_n17408.md")


def measured_traffic():
    """HBM bytes per M=8 launch from the committed rocprofv3 summary, or None."""
    try:
        with open(PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


# Set by --profile-timed: the matmul is then dispatched only as graph replays (no eager
# warm-up calls, no untimed pre-pass), so a kernel trace's per-kernel statistics cover the
# same dispatches the HIP events time.
GRAPH_ONLY = False


def stats(per_call):
    """median / mean / p10 / p90 (us) of per-call times, one per replay."""
    import numpy as np
    a = np.asarray(per_call, dtype=np.float64)
    return {"median": float(np.median(a)), "mean": float(a.mean()),
            "p10": float(np.percentile(a, 10)),
            "p90": float(np.percentile(a, 90)), "replays": int(a.size)}


def replays_for(steps):
    """Replays of a graph (of at least MIN_CALLS_PER_GRAPH calls): 10."""
    return 10


def algorithmic_bytes(M, N=N_OUT, K=K_IN, bits=BITS, gs=GS):
    return N * K * bits // 8 + 2 * N * (K // gs) * 2 + M * K * 2 + M * N * 2


def make_sets(torch, nsets, N, K, bits, gs, dev, seed=1, dtype=None, scale_sd=0.02):
    """`nsets` weight sets of uniform random codes, scales |N(0, scale_sd)| and biases
    N(0, 0.01) in `dtype` (bf16 by default)."""
    dtype = dtype or torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    sets = []
    for _ in range(nsets):
        w = torch.randint(-(2 ** 31), 2 ** 31 - 1, (N, K * bits // 32), dtype=torch.int32,
                          device=dev, generator=g)
        s = (torch.randn(N, K // gs, device=dev, generator=g) * scale_sd).abs().to(dtype)
        b = (torch.randn(N, K // gs, device=dev, generator=g) * 0.01).to(dtype)
        sets.append((w, s, b))
    return sets


def time_replays(torch, stream, graph, steps, reps):
    """Per-call microseconds of `reps` back-to-back replays of a `steps`-call graph, each
    bracketed by HIP events on the graph's stream."""
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
    torch.cuda.synchronize()
    for e0, e1 in events:
        e0.record(stream)
        graph.launch(stream)
        e1.record(stream)
    torch.cuda.synchronize()
    return [e0.elapsed_time(e1) * 1000.0 / steps for e0, e1 in events]


# Fewest calls one timed graph holds.  Each replay's boundary (the graph launch) costs the
# calls around it time that is not the kernel's: measured on MI355X with 24 calls a graph
# against 200 (us per call, same box): the headline M=1 14.96 against 14.53, M=8 15.18-15.40
# against 15.00-15.07, C1 7.03-7.14 against 6.84, C3 17.63 against 16.02-16.17.
MIN_CALLS_PER_GRAPH = 200


def rotation(nsets, steps, set_bytes):
    """The calls one graph captures over `nsets` rotated weight sets of `set_bytes` each: the
    fewest whole cycles through every set that hold at least max(steps, MIN_CALLS_PER_GRAPH)
    calls, so that every set is used equally often and the bytes read between two uses of one
    set -- within a replay and across the boundary into the next replay, which starts again at
    set 0 -- are always (nsets - 1) * set_bytes."""
    calls = -(-max(1, steps, MIN_CALLS_PER_GRAPH) // nsets) * nsets
    return {"calls_per_graph": calls, "sets_touched": nsets,
            "min_reuse_bytes": (nsets - 1) * set_bytes}


def set_bytes_of(sets):
    w, s, b = sets[0]
    return sum(t.numel() * t.element_size() for t in (w, s, b))


def time_m(torch, ctx, stream, sets, M, steps, warmup, N, K, bits, gs, ws, wsb, f16=False,
           x_sd=1.0, packed=None):
    """Per-call microseconds (one figure per replay) of graph-replayed calls at row count M
    (fp16 throughout with f16, else bf16): the graph holds rotation(...)["calls_per_graph"]
    calls (at least `steps` and MIN_CALLS_PER_GRAPH), cycling through every weight set;
    replays_for(steps) replays, each divided by the calls it holds.  With `packed` (the sets in the packed layout,
    Context.pack), the calls are dfq_qmm_packed over those instead."""
    import dflash_qmm
    dev = sets[0][0].device
    g = torch.Generator(device=dev)
    g.manual_seed(100 + M)
    tdt = torch.float16 if f16 else torch.bfloat16
    x = (torch.randn(M, K, device=dev, generator=g) * x_sd).to(tdt)
    y = torch.empty(M, N, device=dev, dtype=tdt)
    B = dflash_qmm.F16 if f16 else dflash_qmm.BF16

    def issue(count, start):
        for i in range(count):
            if packed is not None:
                ctx.qmm_packed_raw(x, packed[(start + i) % len(packed)], y, M, ws=ws,
                                   ws_bytes=wsb, stream=stream)
                continue
            w, s, b = sets[(start + i) % len(sets)]
            ctx.qmm_raw(x, w, s, b, y, M, N, K, bits, gs, B, B, B, ws=ws, ws_bytes=wsb,
                        stream=stream)

    calls = rotation(len(sets), steps, 0)["calls_per_graph"]
    torch.cuda.synchronize()
    ctx.graph_begin(stream)
    issue(calls, 0)
    graph = ctx.graph_end(stream)
    with torch.cuda.stream(stream):
        if not GRAPH_ONLY:
            issue(warmup, 1)           # eager warm-up (also checks the eager path)
        graph.launch(stream)           # graph warm-up
        times = time_replays(torch, stream, graph, calls, replays_for(steps))
    graph.close()
    return times


# The other benchmark configurations, timed like the headline (one graph of `steps` calls,
# replays_for(steps) replays, weights rotated over enough sets to exceed the 256 MB
# Infinity Cache): (name, M, N, K, bits, group, fp16, x standard deviation, scale sd).
CONFIGS = [
    ("c1_m1_k4096_n4096_b4g64_f16", 1, 4096, 4096, 4, 64, True, 1.0, 0.02),
    ("c3_down_m8_k17408_n5120_b4g64", 8, 5120, 17408, 4, 64, False, 0.5, 0.02),
    ("c4_qkv_m8_k5120_n7168_b8g64", 8, 7168, 5120, 8, 64, False, 1.0, 0.004),
    ("c4_o_m8_k5120_n5120_b8g64", 8, 5120, 5120, 8, 64, False, 1.0, 0.004),
    ("c4_qkv_m8_k5120_n7168_b4g32", 8, 7168, 5120, 4, 32, False, 1.0, 0.02),
    ("c4_o_m8_k5120_n5120_b4g32", 8, 5120, 5120, 4, 32, False, 1.0, 0.02),
]


def time_configs(torch, ctx, stream, dev, steps, warmup):
    """Median per-call us, GB/s and fraction of 8 TB/s for each of CONFIGS."""
    out = {}
    for (name, M, N, K, bits, gs, f16, x_sd, s_sd) in CONFIGS:
        nb = algorithmic_bytes(M, N, K, bits, gs)
        nsets = max(2, -(-400_000_000 // algorithmic_bytes(0, N, K, bits, gs)))
        sets = make_sets(torch, nsets, N, K, bits, gs, dev, seed=3,
                         dtype=torch.float16 if f16 else torch.bfloat16, scale_sd=s_sd)
        wsb = ctx.workspace_bytes(M, N, K, bits, gs)
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
        d = stats(time_m(torch, ctx, stream, sets, M, steps, warmup, N, K, bits, gs, ws,
                         ws.numel(), f16=f16, x_sd=x_sd))
        if M == 1:  # below the window: the stock path a swapped layer takes at one row
            stock1 = time_stock(torch, ctx, stream, sets, [1], N, K, bits, gs, f16,
                                steps=steps)["1"]
        out[name] = {"us_per_call": round(d["median"], 3), "p10": round(d["p10"], 3),
                     "p90": round(d["p90"], 3), "bytes": nb,
                     "gbs": round(nb / (d["median"] * 1e-6) / 1e9, 1),
                     "frac": round(nb / (d["median"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "rotated_sets": nsets,
                     **rotation(nsets, steps, set_bytes_of(sets))}
        if M == 1:
            out[name]["stock_us_per_call"] = stock1
            out[name]["stock_gbs"] = round(nb / (stock1 * 1e-6) / 1e9, 1)
        print(f"[bench] {name}: {d['median']:.2f} us/call, {out[name]['gbs']:.0f} GB/s",
              file=sys.stderr, flush=True)
        del sets
    return out


def time_read(torch, ctx, stream, nbytes, nsets, steps, dev):
    """The read ceiling: the plain streaming-read kernel over `nsets` rotated buffers of
    `nbytes`, `steps` launches per graph, replayed like the matmul; per-launch us."""
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(nsets)]
    sink = torch.zeros(8 * ctx.num_cus, dtype=torch.int32, device=dev)
    calls = rotation(nsets, steps, nbytes)["calls_per_graph"]
    torch.cuda.synchronize()
    ctx.graph_begin(stream)
    for i in range(calls):
        ctx.read_stream(bufs[i % nsets], nbytes, sink, stream=stream)
    graph = ctx.graph_end(stream)
    with torch.cuda.stream(stream):
        graph.launch(stream)
        times = time_replays(torch, stream, graph, calls, replays_for(steps))
    graph.close()
    return times


def time_units(torch, ctx, stream, sets, M, steps, N=N_OUT, K=K_IN, packed=None):
    """The fast kernel's own loads with no compute (dfq_debug_read_units, or
    dfq_debug_read_units_packed over `packed`) over the rotated weight sets of the matmul,
    `steps` launches per graph, replayed like it; per-launch us."""
    sink = torch.zeros(12 * ctx.num_cus, dtype=torch.int32, device=sets[0][0].device)
    calls = rotation(len(sets), steps, 0)["calls_per_graph"]
    torch.cuda.synchronize()
    ctx.graph_begin(stream)
    for i in range(calls):
        if packed is not None:
            ctx.read_units_packed(packed[i % len(packed)].data, M, N, K, sink, stream=stream)
            continue
        w, s, b = sets[i % len(sets)]
        ctx.read_units(w, s, b, M, N, K, sink, stream=stream)
    graph = ctx.graph_end(stream)
    with torch.cuda.stream(stream):
        graph.launch(stream)
        times = time_replays(torch, stream, graph, calls, replays_for(steps))
    graph.close()
    return times


def time_stock(torch, ctx, stream, sets, rows, N=N_OUT, K=K_IN, bits=BITS, gs=GS, f16=False,
               steps=20, reps=10):
    """The stock path a swapped layer falls through to (dfq_qmm_fallback: its GEMV, one launch
    per 4 rows) at each of `rows`, over the rotated weight sets, timed like the fast kernel;
    median per-call us."""
    import dflash_qmm
    dev = sets[0][0].device
    B = dflash_qmm.F16 if f16 else dflash_qmm.BF16
    tdt = torch.float16 if f16 else torch.bfloat16
    calls = rotation(len(sets), steps, 0)["calls_per_graph"]
    out = {}
    for M in rows:
        g = torch.Generator(device=dev)
        g.manual_seed(100 + M)
        x = torch.randn(M, K, device=dev, generator=g).to(tdt)
        y = torch.empty(M, N, device=dev, dtype=tdt)
        torch.cuda.synchronize()
        ctx.graph_begin(stream)
        for i in range(calls):
            w, s, b = sets[i % len(sets)]
            ctx.fallback_raw(x, w, s, b, y, M, N, K, bits, gs, B, B, B, stream=stream)
        graph = ctx.graph_end(stream)
        with torch.cuda.stream(stream):
            graph.launch(stream)
            d = stats(time_replays(torch, stream, graph, calls, reps))
        graph.close()
        out[str(M)] = round(d["median"], 3)
        print(f"[bench] stock M={M} N={N} K={K}: {d['median']:.2f} us/call", file=sys.stderr,
              flush=True)
    return out


def time_copy(torch, stream, nbytes, nsets, steps):
    """A plain device copy moving `nbytes` per launch (nbytes/2 read, nbytes/2 written),
    rotated over buffers larger than the Infinity Cache and timed back to back like the
    matmul: the launch-for-launch bandwidth a memory-bound kernel of this size reaches on
    this GPU.  Microseconds per copy."""
    dev = torch.device("cuda:0")
    half = nbytes // 2
    src = [torch.ones(half, dtype=torch.uint8, device=dev) for _ in range(nsets)]
    dst = [torch.empty(half, dtype=torch.uint8, device=dev) for _ in range(nsets)]
    with torch.cuda.stream(stream):
        for i in range(20):
            dst[i % nsets].copy_(src[(i + 1) % nsets])
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        calls = max(steps, MIN_CALLS_PER_GRAPH)
        e0.record(stream)
        for i in range(calls):
            dst[i % nsets].copy_(src[(i + 1) % nsets])
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / calls


# One verify-pass layer of the C5 chain (N, K): q, k, v, o, gate, up, down; then the lm_head.
C5_LAYER = [(5120, 5120), (1024, 5120), (1024, 5120), (5120, 5120), (17408, 5120),
            (17408, 5120), (5120, 17408)]
# The same layer with the projections that read one input fused (weights concatenated at
# load): q|k|v, o, gate|up (then SiLU-mul on the device), down.
C5_FUSED = [(7168, 5120), (5120, 5120), (34816, 5120), (5120, 17408)]
C5_LM_HEAD = (151936, 5120)


def c5_weights(torch, dev, fused, layers=64):
    """Distinct random 4-bit g64 weights for every layer of the C5 verify forward (about
    11.6 GiB, so every layer streams from HBM) and the LM head: codes uniform, scales
    |N(0, 0.02)|, biases N(0, 0.01), bf16.  Fused: q|k|v, o, gate|up (interleaved by 8 rows
    for the SiLU-mul epilogue), down; else the seven projections."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)

    def weights(N, K):
        w = torch.randint(-(2 ** 31), 2 ** 31 - 1, (N, K // 8), dtype=torch.int32, device=dev,
                          generator=g)
        s = (torch.randn(N, K // 64, device=dev, generator=g) * 0.02).abs().to(torch.bfloat16)
        b = (torch.randn(N, K // 64, device=dev, generator=g) * 0.01).to(torch.bfloat16)
        return w, s, b

    layer = C5_FUSED if fused else C5_LAYER
    return {"fused": fused, "layers": layers, "layer": layer,
            "lw": [[weights(N, K) for (N, K) in layer] for _ in range(layers)],
            "lm": weights(*C5_LM_HEAD)}


def pack_c5(ctx, W):
    """The same weights in the packed layout (Context.pack), for the packed forward."""
    return {**W, "packed": True,
            "lw": [[ctx.pack(w, s, b, 4, 64) for (w, s, b) in lw] for lw in W["lw"]],
            "lm": ctx.pack(*W["lm"], 4, 64)}


C5_FORMS = {
    "per_layer": "one HIP graph per layer, launched one after the other",
    "composed": "one HIP graph per layer, the 64 composed into one launch (dfq_graph_compose)",
    "one_graph": "the forward captured as one HIP graph",
}


def chain_c5(torch, ctx, dev, W, M=8, form="per_layer", forwards=10):
    """The C5 verify forward at M rows over the weights W (c5_weights): every layer's
    projections, then the LM head with the greedy accept (only M + 1 ints leave the device).
    Each layer is captured as one HIP graph (the configuration's form); `form` says how the
    forward launches them (C5_FORMS).  One untimed forward, then `forwards` timed ones, each
    between its own HIP events; figures are the median with p10 / p90."""
    import dflash_qmm
    fused, layers, layer = W["fused"], W["layers"], W["layer"]
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    shapes = layer + [C5_LM_HEAD]
    wsb = max(ctx.workspace_bytes(M, N, K, 4, 64) for (N, K) in shapes)
    ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
    x = torch.randn(M, 5120, device=dev, generator=g).to(torch.bfloat16)
    if fused:
        # q|k|v, o and gate|up read the layer input (o stands in for attention's output);
        # gate|up (weights interleaved by 8 rows) writes silu(gate) * up; down reads it
        outs = [torch.empty(M, N // 2 if j == 2 else N, device=dev, dtype=torch.bfloat16)
                for j, (N, K) in enumerate(layer)]
        srcs = [None, None, None, 2]
        kinds = ["qmm", "qmm", "qmm_silu_gate_up", "qmm"]
    else:
        # q, k, v, gate, up read x (the layer input); o reads q; down reads gate
        outs = [torch.empty(M, N, device=dev, dtype=torch.bfloat16) for (N, K) in layer]
        srcs = [None, None, None, 0, None, None, 4]
        kinds = ["qmm"] * len(layer)
    stream = torch.cuda.Stream(device=dev)
    B = dflash_qmm.BF16
    packed = W.get("packed", False)
    proposals = torch.zeros(max(1, M - 1), dtype=torch.int32, device=dev)
    tokens = torch.empty(M, dtype=torch.int32, device=dev)
    accepted = torch.empty(1, dtype=torch.int32, device=dev)
    acc_ws = torch.zeros(ctx.qmm_argmax_accept_workspace_bytes(M, *C5_LM_HEAD, 4, 64),
                         dtype=torch.uint8, device=dev)

    def enqueue_layer(li):
        wl = W["lw"][li]
        layer_in = x if li == 0 else outs[-1]
        for j, (N, K) in enumerate(layer):
            inp = layer_in if srcs[j] is None else outs[srcs[j]]
            if packed:
                if kinds[j] == "qmm_silu_gate_up":
                    ctx.qmm_silu_gate_up_packed(inp, wl[j], out=outs[j], ws=ws, stream=stream)
                else:
                    ctx.qmm_packed_raw(inp, wl[j], outs[j], M, ws=ws, ws_bytes=ws.numel(),
                                       stream=stream)
                continue
            w, s, b = wl[j]
            if kinds[j] == "qmm_silu_gate_up":
                ctx.qmm_silu_gate_up(inp, w, s, b, 4, 64, out=outs[j], ws=ws, stream=stream)
            else:
                ctx.qmm_raw(inp, w, s, b, outs[j], M, N, K, 4, 64, B, B, B, ws=ws,
                            ws_bytes=ws.numel(), stream=stream)

    def lm_only():
        if packed:
            ctx.qmm_argmax_accept_packed(outs[-1], W["lm"],
                                         proposals=proposals if M > 1 else None, tokens=tokens,
                                         accepted=accepted, ws=acc_ws, stream=stream)
            return
        wlm, slm, blm = W["lm"]
        ctx.qmm_argmax_accept(outs[-1], wlm, slm, blm, 4, 64,
                              proposals=proposals if M > 1 else None, tokens=tokens,
                              accepted=accepted, ws=acc_ws, stream=stream)

    torch.cuda.synchronize()
    graphs, launch = [], []
    if form == "one_graph":
        ctx.graph_begin(stream)
        for li in range(layers):
            enqueue_layer(li)
        lm_only()
        launch = [ctx.graph_end(stream)]
    else:
        for li in range(layers):
            ctx.graph_begin(stream)
            enqueue_layer(li)
            graphs.append(ctx.graph_end(stream))
        launch = [ctx.graph_compose(graphs)] if form == "composed" else graphs

    def forward():
        for gr in launch:
            gr.launch(stream)
        if form != "one_graph":
            lm_only()

    def timed(fn, n):
        with torch.cuda.stream(stream):
            fn()
            torch.cuda.synchronize()
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(n)]
            for e0, e1 in ev:
                e0.record(stream)
                fn()
                e1.record(stream)
            torch.cuda.synchronize()
        return [e0.elapsed_time(e1) * 1000.0 for e0, e1 in ev]

    fw = stats(timed(forward, forwards))
    lm = stats(timed(lm_only, 20))
    for gr in set(graphs) | set(launch):
        gr.close()
    layer_bytes = sum(algorithmic_bytes(M, N, K) for (N, K) in C5_LAYER)   # the same fused
    total_bytes = layers * layer_bytes + algorithmic_bytes(M, *C5_LM_HEAD)
    ideal = total_bytes / (HBM_PEAK_GBS * 1e3)
    total = fw["median"]
    return {
        "workload": (f"M={M} verify forward: {layers} layers x "
                     + ("(q|k|v, o, gate|up with silu*up epilogue, down)" if fused
                        else "(q,k,v,o,gate,up,down)")
                     + " + lm_head + greedy accept, 4-bit g64 bf16"
                     + (" in the packed layout" if packed else "") + ", " + C5_FORMS[form]),
        "us_per_forward": round(total, 1),
        "p10": round(fw["p10"], 1),
        "p90": round(fw["p90"], 1),
        "forwards": fw["replays"],
        "ideal_us_at_8TBs": round(ideal, 1),
        "frac_of_ideal": round(ideal / total, 4),
        "bytes_per_forward": total_bytes,
        "layer_us": round((total - lm["median"]) / layers, 2),
        "layer_ideal_us": round(layer_bytes / (HBM_PEAK_GBS * 1e3), 2),
        "lm_head_accept_us": round(lm["median"], 2),
        "lm_head_ideal_us": round(algorithmic_bytes(M, *C5_LM_HEAD) / (HBM_PEAK_GBS * 1e3), 2),
    }


# Verify widths of the forward-cost curve (the reference's dflash-bench --rows sweep).
C5_ROWS = [1, 2, 4, 5, 6, 8, 9, 12, 16]


def c5_rows(torch, ctx, dev, W, rows=C5_ROWS, form="composed", forwards=10):
    """The fused verify forward's cost at each verify width, and its ratio to one row."""
    out = {}
    for M in rows:
        r = chain_c5(torch, ctx, dev, W, M=M, form=form, forwards=forwards)
        out[str(M)] = {"us_per_forward": r["us_per_forward"], "p10": r["p10"], "p90": r["p90"]}
        print(f"[bench] c5 rows M={M}: {r['us_per_forward']} us/forward", file=sys.stderr,
              flush=True)
    base = out[str(rows[0])]["us_per_forward"]
    for M in rows:
        out[str(M)]["ratio_to_m1"] = round(out[str(M)]["us_per_forward"] / base, 4)
    return {"workload": ("fused verify forward (64 layers + LM head + greedy accept, 4-bit g64 "
                         "bf16), " + C5_FORMS[form] + f", median of {forwards} forwards per width"),
            "rows": out}


def time_lm_head(torch, ctx, stream, dev, steps=20, nsets=4, reps=20):
    """The C5 LM head (M=8, 151936 x 5120, 4-bit g64) with the greedy accept, graph-replayed
    over rotated weights: fused (dfq_qmm_argmax_accept, no logits written) and as two calls
    (dfq_qmm to logits, then dfq_argmax_accept).  Per-call us."""
    import dflash_qmm
    M, (V, K) = 8, C5_LM_HEAD
    sets = make_sets(torch, nsets, V, K, 4, 64, dev, seed=9)
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    logits = torch.empty(M, V, device=dev, dtype=torch.bfloat16)
    props = torch.zeros(M - 1, dtype=torch.int32, device=dev)
    tokens = torch.empty(M, dtype=torch.int32, device=dev)
    acc = torch.empty(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(max(ctx.qmm_argmax_accept_workspace_bytes(M, V, K, 4, 64),
                         ctx.workspace_bytes(M, V, K, 4, 64)), dtype=torch.uint8, device=dev)
    acc_ws = torch.zeros(256, dtype=torch.uint8, device=dev)
    B = dflash_qmm.BF16
    packed = [ctx.pack(w, s, b, 4, 64) for (w, s, b) in sets]
    out = {}
    for form in ("fused", "fused_packed", "two_calls"):
        torch.cuda.synchronize()
        ctx.graph_begin(stream)
        for i in range(steps):
            w, s, b = sets[i % nsets]
            if form == "fused_packed":
                ctx.qmm_argmax_accept_packed(x, packed[i % nsets], proposals=props,
                                             tokens=tokens, accepted=acc, ws=ws, stream=stream)
            elif form == "fused":
                ctx.qmm_argmax_accept(x, w, s, b, 4, 64, proposals=props, tokens=tokens,
                                      accepted=acc, ws=ws, stream=stream)
            else:
                ctx.qmm_raw(x, w, s, b, logits, M, V, K, 4, 64, B, B, B, ws=ws,
                            ws_bytes=ws.numel(), stream=stream)
                ctx.argmax_accept(logits, props, tokens, acc, ws=acc_ws, stream=stream)
        graph = ctx.graph_end(stream)
        with torch.cuda.stream(stream):
            graph.launch(stream)
            out[form] = stats(time_replays(torch, stream, graph, steps, reps))["median"]
        graph.close()
    nb = algorithmic_bytes(M, V, K)
    return {
        "workload": ("LM head M=8, 151936 x 5120 4-bit g64 bf16, with the greedy accept; "
                     f"{nsets} rotated weight sets ({nsets * 440} MB), median of {reps} "
                     f"replays of {steps} calls"),
        "fused_us": round(out["fused"], 2),
        "fused_packed_us": round(out["fused_packed"], 2),
        "two_calls_us": round(out["two_calls"], 2),
        "ideal_us_at_8TBs": round(nb / (HBM_PEAK_GBS * 1e3), 2),
        "fused_gbs": round(nb / (out["fused"] * 1e-6) / 1e9, 1),
    }


def cpu_baseline(seconds):
    """The oracle's OpenMP fp32 restatement on a bounded sample of the M=8 workload."""
    import numpy as np
    from oracle.qmm_oracle import COracle, make_case
    orc = COracle()
    n_sample = 2048
    c = make_case(8, n_sample, K_IN, bits=BITS, gs=GS, seed=5)
    orc.qmm_f32(c)  # warm
    calls, t0 = 0, time.perf_counter()
    while True:
        orc.qmm_f32(c)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per_call_sample = el / calls
    per_call_full = per_call_sample * (N_OUT / n_sample)  # rows are independent
    us = per_call_full * 1e6
    return {
        "value": round(algorithmic_bytes(8) / per_call_full / 1e9, 3),
        "unit": "GB/s",
        "us_per_call": round(us, 1),
        "cores": orc.num_threads(),
        "kind": "port",
        "label": "MLX-semantics CPU restatement, not MLX",
        "sample": (f"M=8 K=5120 4-bit g64 bf16, {n_sample} of 17408 output rows, {calls} calls "
                   f"in {el:.1f}s, scaled to all rows"),
    }


def trace_summary(path, steps):
    """Per-dispatch kernel durations (ns) from a rocprofv3 kernel-trace CSV of a
    --profile-timed run, per dfq_qmm kernel in dispatch order: its first `steps` dispatches
    are the warm-up replay, the rest the timed replays."""
    import csv
    import numpy as np
    runs = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Kernel_Name"].startswith("dfq_qmm"):
                runs.setdefault(r["Kernel_Name"], []).append(
                    (int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    out = {}
    for name, ev in runs.items():
        ev.sort()
        d = np.array([e - s for s, e in ev], dtype=np.float64)

        def st(a):
            if not a.size:
                return None
            return {"dispatches": int(a.size), "mean": round(float(a.mean()), 1),
                    "median": round(float(np.median(a)), 1),
                    "p10": round(float(np.percentile(a, 10)), 1),
                    "p90": round(float(np.percentile(a, 90)), 1)}
        out[name] = {"all": st(d), "warmup_replay": st(d[:steps]), "timed": st(d[steps:])}
    return out


def c5_trace_summary(path, layers=64):
    """Per-op kernel durations of the timed verify forwards in a rocprofv3 kernel-trace CSV
    of `bench.py --c5-only ...`.  A forward ends with the LM head's greedy-accept dispatch;
    the first forward (the warm-up) and the LM-head-only calls after the forwards are left
    out.  Per position within a layer: the kernel, its mean duration and the mean gap before
    it (us)."""
    import csv
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Kernel_Name"].startswith("dfq_"):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                             r["Kernel_Name"]))
    rows.sort()
    ends = [i for i, r in enumerate(rows) if r[2].endswith("_am") or "argmax_accept" in r[2]]
    fwds, tail = [], 0
    for i0, i1 in zip(ends, ends[1:]):
        seg = rows[i0 + 1:i1 + 1]
        # the LM head's dispatches: the fused head, or the head, its second pass and the
        # accept (splits with a second pass)
        for tl in (1, 2, 3):
            if len(seg) >= layers + tl and (len(seg) - tl) % layers == 0:
                fwds.append(seg)
                tail = tl
                break
    if not fwds:
        return {"forwards": 0}
    fwds = [seg for seg in fwds if len(seg) == len(fwds[0])]
    per = (len(fwds[0]) - tail) // layers
    ops = []
    for j in range(per + tail):
        dur, gap = [], []
        for seg in fwds:
            idx = ([j + per * li for li in range(layers)] if j < per
                   else [len(seg) - tail + (j - per)])
            for i in idx:
                dur.append(seg[i][1] - seg[i][0])
                if i:
                    gap.append(seg[i][0] - seg[i - 1][1])
        name = fwds[0][j][2] if j < per else fwds[0][len(fwds[0]) - tail + (j - per)][2]
        ops.append({"kernel": name, "mean_us": round(sum(dur) / len(dur) / 1e3, 2),
                    "gap_before_us": round(sum(gap) / max(1, len(gap)) / 1e3, 2)})
    spans = [(seg[-1][1] - seg[0][0]) / 1e3 for seg in fwds]
    return {"forwards": len(fwds), "dispatches_per_forward": len(fwds[0]),
            "span_us_per_forward": [round(v, 1) for v in spans], "ops": ops}


def main():
    global GRAPH_ONLY
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sets", type=int, default=8, help="rotated weight sets")
    ap.add_argument("--ms", default="1,2,3,4,5,6,8,12,16")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-chain", action="store_true",
                    help="skip the 64-layer verify-forward measurement (c5_chain)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other benchmark configurations (C1, C3, C4)")
    ap.add_argument("--no-reference", action="store_true",
                    help="skip the read-ceiling and device-copy reference legs")
    ap.add_argument("--no-stock", action="store_true",
                    help="skip the stock path's timing beside the fast kernel")
    ap.add_argument("--no-rows", action="store_true",
                    help="skip the verify forward's cost at each width (c5_rows)")
    ap.add_argument("--no-packed", action="store_true",
                    help="skip the packed-layout legs (dfq_qmm_packed and its fused forms)")
    ap.add_argument("--c5-only", choices=["separate", "fused", "fused_composed",
                                          "fused_one_graph", "fused_composed_packed"],
                    default=None,
                    help="only time this form of the 64-layer verify forward (for profiling) "
                         "and print its figures")
    ap.add_argument("--c5-m", type=int, default=8,
                    help="rows of the verify forward that --c5-only times (1..16)")
    ap.add_argument("--shape", metavar="M,N,K,BITS,GS[,f16]", default=None,
                    help="time only this call, rotated over enough weight sets to exceed the "
                         "Infinity Cache and replayed like the headline, print its figures and "
                         "exit (with --profile-timed, for a kernel trace of one shape)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run 20 plain device copies of this many MiB (the reference "
                         "point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--profile-timed", action="store_true",
                    help="dispatch the matmul only as graph replays, so that a kernel "
                         "trace covers the timed calls (plus one warm-up replay)")
    ap.add_argument("--c5-trace-summary", metavar="CSV", default=None,
                    help="summarise the run_kernel_trace.csv of a --c5-only rocprofv3 run "
                         "(per-op durations of the timed forwards) and exit; needs no GPU")
    ap.add_argument("--trace-summary", metavar="CSV", default=None,
                    help="summarise the run_kernel_trace.csv of a --profile-timed rocprofv3 "
                         "run (per-dispatch durations of each dfq_qmm kernel, the warm-up "
                         "replay apart from the timed replays) and exit; needs no GPU")
    args = ap.parse_args()

    if args.c5_trace_summary:
        print(json.dumps(c5_trace_summary(args.c5_trace_summary)), flush=True)
        return
    if args.trace_summary:
        print(json.dumps(trace_summary(args.trace_summary, args.steps)), flush=True)
        return

    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the matmul path runs on a single GPU)", file=sys.stderr)
        sys.exit(2)

    import torch
    import dflash_qmm

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    GRAPH_ONLY = args.profile_timed
    dev = torch.device("cuda:0")
    if args.copy_mib:
        n = args.copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n, "launches": 20}), flush=True)
        return
    ctx = dflash_qmm.Context(0)
    if args.shape:
        parts = args.shape.split(",")
        M, N, K, bits, gs = (int(v) for v in parts[:5])
        f16 = len(parts) > 5 and parts[5] == "f16"
        nsets = max(2, -(-400_000_000 // algorithmic_bytes(0, N, K, bits, gs)))
        sets = make_sets(torch, nsets, N, K, bits, gs, dev, seed=3,
                         dtype=torch.float16 if f16 else torch.bfloat16,
                         scale_sd=0.02 if bits == 4 else 0.004)
        wsb = ctx.workspace_bytes(M, N, K, bits, gs)
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
        stream = torch.cuda.Stream(device=dev)
        d = stats(time_m(torch, ctx, stream, sets, M, args.steps, args.warmup, N, K, bits, gs,
                         ws, ws.numel(), f16=f16))
        nb = algorithmic_bytes(M, N, K, bits, gs)
        print(json.dumps({"shape": {"M": M, "N": N, "K": K, "bits": bits, "group_size": gs,
                                    "dtype": "f16" if f16 else "bf16"},
                          "us_per_call": round(d["median"], 3), "p10": round(d["p10"], 3),
                          "p90": round(d["p90"], 3), "replays": d["replays"],
                          "bytes": nb, "gbs": round(nb / (d["median"] * 1e-6) / 1e9, 1),
                          "frac": round(nb / (d["median"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "rotated_sets": nsets, **rotation(nsets, args.steps,
                                                            set_bytes_of(sets))}), flush=True)
        ctx.close()
        return
    if args.c5_only:
        fused = args.c5_only.startswith("fused")
        form = {"separate": "per_layer", "fused": "per_layer", "fused_composed": "composed",
                "fused_one_graph": "one_graph",
                "fused_composed_packed": "composed"}[args.c5_only]
        W = c5_weights(torch, dev, fused)
        if args.c5_only.endswith("_packed"):
            W = pack_c5(ctx, W)
        r = chain_c5(torch, ctx, dev, W, M=args.c5_m, form=form)
        print(json.dumps({"c5_" + args.c5_only: r}), flush=True)
        ctx.close()
        return
    stream = torch.cuda.Stream(device=dev)
    sets = make_sets(torch, args.sets, N_OUT, K_IN, BITS, GS, dev)
    ms = [int(v) for v in args.ms.split(",")]
    if 8 not in ms:
        ms.append(8)
    wsb = max(ctx.workspace_bytes(m, N_OUT, K_IN, BITS, GS) for m in ms)
    ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)

    torch.cuda.synchronize()
    # one untimed pass first: the first M timed on a cold GPU otherwise reads up to ~1 us slow
    if not GRAPH_ONLY:
        time_m(torch, ctx, stream, sets, ms[0], args.steps, args.warmup, N_OUT, K_IN, BITS, GS,
               ws, ws.numel())
    dist = {}
    for m in ms:
        dist[m] = stats(time_m(torch, ctx, stream, sets, m, args.steps, args.warmup, N_OUT,
                               K_IN, BITS, GS, ws, ws.numel()))
        d = dist[m]
        print(f"[bench] M={m}: {d['median']:.2f} us/call (mean {d['mean']:.2f}, p10 "
              f"{d['p10']:.2f}, p90 "
              f"{d['p90']:.2f}, {d['replays']} replays of "
              f"{rotation(args.sets, args.steps, 0)['calls_per_graph']}), "
              f"{algorithmic_bytes(m) / d['median'] / 1e3:.0f} GB/s", file=sys.stderr,
              flush=True)
    us = {m: dist[m]["median"] for m in ms}
    gbs = {m: algorithmic_bytes(m) / (us[m] * 1e-6) / 1e9 for m in ms}
    achieved = gbs[8]
    nb8 = algorithmic_bytes(8)
    out = {
        "metric": "us/call + HBM GB/s, 4-bit qmatmul K5120xN17408, M=1..8; M8/M1 time ratio",
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us[8] / 1000.0, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "affine qmm 4-bit g64, K=5120, N=17408, bf16, M=8 per step",
            "M_sweep": ms,
            "rotated_weight_sets": args.sets,
            "replays_per_M": replays_for(args.steps),
            "min_calls_per_graph": MIN_CALLS_PER_GRAPH,
            "rotation": rotation(args.sets, args.steps, set_bytes_of(sets)),
            "mall_bytes": MALL_BYTES,
        },
        "us_per_call": {str(m): round(us[m], 3) for m in ms},
        "us_per_call_p10": {str(m): round(dist[m]["p10"], 3) for m in ms},
        "us_per_call_p90": {str(m): round(dist[m]["p90"], 3) for m in ms},
        "gbs_by_M": {str(m): round(gbs[m], 1) for m in ms},
        "m8_m1_ratio": round(us[8] / us[1], 4) if 1 in us else None,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
        },
    }
    if not args.no_reference:
        rd = stats(time_read(torch, ctx, stream, nb8, args.sets, args.steps, dev))
        out["read_ceiling"] = {
            "workload": ("the library's plain streaming-read kernel (one workgroup of 8 waves "
                         "per CU, 4 KB blocks dealt to the waves round-robin, 32 KB in flight "
                         "per CU) reading the M=8 call's algorithmic bytes per launch, rotated "
                         "over buffers, replayed like the matmul"),
            "bytes_per_launch": nb8,
            "us_per_launch": round(rd["median"], 3),
            "p10": round(rd["p10"], 3),
            "p90": round(rd["p90"], 3),
            "gbs": round(nb8 / (rd["median"] * 1e-6) / 1e9, 1),
            "matmul_frac_of_ceiling": round(rd["median"] / us[8], 4),
        }
        print(f"[bench] read ceiling {nb8 / 1e6:.1f} MB: {rd['median']:.2f} us/launch, "
              f"{nb8 / rd['median'] / 1e3:.0f} GB/s", file=sys.stderr, flush=True)
        ud = stats(time_units(torch, ctx, stream, sets, 8, args.steps))
        wb = algorithmic_bytes(0)  # weights, scales and biases
        out["unit_read"] = {
            "workload": ("the fast kernel's own loads for M=8 with no compute "
                         "(dfq_debug_read_units: its workgroup ranges, one unit of 16 columns x "
                         "512 k in flight per wave, 12 waves per CU), over the same rotated "
                         "weight sets"),
            "bytes_per_launch": wb,
            "us_per_launch": round(ud["median"], 3),
            "p10": round(ud["p10"], 3),
            "p90": round(ud["p90"], 3),
            "gbs": round(wb / (ud["median"] * 1e-6) / 1e9, 1),
            "matmul_frac_of_unit_read": round(ud["median"] / us[8], 4),
        }
        print(f"[bench] the kernel's own loads without compute: {ud['median']:.2f} us/launch",
              file=sys.stderr, flush=True)
        uc_copy = time_copy(torch, stream, nb8, args.sets, args.steps)
        out["device_copy"] = {
            "workload": ("torch copy_ of half the M=8 call's algorithmic bytes into another "
                         "buffer (the same bytes moved per launch), rotated, back to back"),
            "bytes_per_launch": nb8,
            "us_per_copy": round(uc_copy, 3),
            "gbs": round(nb8 / (uc_copy * 1e-6) / 1e9, 1),
        }
        print(f"[bench] device copy moving {nb8 / 1e6:.1f} MB: {uc_copy:.2f} us/copy",
              file=sys.stderr, flush=True)
    if not args.no_packed:
        psets = [ctx.pack(w, s, b, BITS, GS) for (w, s, b) in sets]
        pdist = {m: stats(time_m(torch, ctx, stream, sets, m, args.steps, args.warmup, N_OUT,
                                 K_IN, BITS, GS, ws, ws.numel(), packed=psets)) for m in ms}
        pud = stats(time_units(torch, ctx, stream, sets, 8, args.steps, packed=psets))
        pus = {m: pdist[m]["median"] for m in ms}
        out["packed"] = {
            "workload": ("the same calls over the same rotated weight sets in the packed "
                         "layout (dfq_pack_weights once at load, then dfq_qmm_packed): each "
                         "unit of 16 rows x 8 groups is one contiguous piece, its codes in the "
                         "order the lanes load them, then its scales and biases"),
            "us_per_call": {str(m): round(pus[m], 3) for m in ms},
            "us_per_call_p10": {str(m): round(pdist[m]["p10"], 3) for m in ms},
            "us_per_call_p90": {str(m): round(pdist[m]["p90"], 3) for m in ms},
            "gbs_by_M": {str(m): round(algorithmic_bytes(m) / (pus[m] * 1e-6) / 1e9, 1)
                         for m in ms},
            "faster_than_mlx_layout_us": {str(m): round(us[m] - pus[m], 3) for m in ms},
            "unit_read_us": round(pud["median"], 3),
            "unit_read_p10": round(pud["p10"], 3),
            "unit_read_p90": round(pud["p90"], 3),
        }
        print(f"[bench] packed layout: M=8 {pus[8]:.2f} us/call ({us[8] - pus[8]:+.2f} us "
              f"faster), its own loads {pud['median']:.2f} us/launch", file=sys.stderr,
              flush=True)
        del psets
    if not args.no_stock:
        st = time_stock(torch, ctx, stream, sets, [m for m in ms if m <= 8], steps=args.steps)
        out["stock"] = {
            "workload": ("dfq_qmm_fallback, the stock path a swapped layer falls through to "
                         "below the window's lower bound (its GEMV, one launch per 4 rows), "
                         "on the headline shape, rotated and replayed like the fast kernel"),
            "us_per_call": st,
            "fast_us_per_call": {k: round(us[int(k)], 3) for k in st},
            "fast_wins_from_rows": min([int(k) for k in st if us[int(k)] < st[k]], default=None),
        }
    del sets
    torch.cuda.empty_cache()
    if not args.no_configs:
        out["configs"] = time_configs(torch, ctx, stream, dev, args.steps, args.warmup)
        torch.cuda.empty_cache()
    if not args.no_chain:
        out["lm_head_accept"] = time_lm_head(torch, ctx, stream, dev)
        print(f"[bench] lm_head + accept: fused {out['lm_head_accept']['fused_us']} us, two "
              f"calls {out['lm_head_accept']['two_calls_us']} us", file=sys.stderr, flush=True)
        W = c5_weights(torch, dev, fused=False)
        out["c5_chain"] = chain_c5(torch, ctx, dev, W, form="per_layer")
        del W
        torch.cuda.empty_cache()
        W = c5_weights(torch, dev, fused=True)
        for key, form in (("c5_chain_fused", "per_layer"), ("c5_chain_fused_composed", "composed"),
                          ("c5_chain_fused_one_graph", "one_graph")):
            out[key] = chain_c5(torch, ctx, dev, W, form=form)
        for key in ("c5_chain", "c5_chain_fused", "c5_chain_fused_composed",
                    "c5_chain_fused_one_graph"):
            print(f"[bench] {key}: {out[key]['us_per_forward']} us/forward "
                  f"(ideal {out[key]['ideal_us_at_8TBs']})", file=sys.stderr, flush=True)
        if not args.no_rows:
            out["c5_rows"] = c5_rows(torch, ctx, dev, W)
        if not args.no_packed:
            WP = pack_c5(ctx, W)
            for key, form in (("c5_chain_fused_composed_packed", "composed"),
                              ("c5_chain_fused_one_graph_packed", "one_graph")):
                out[key] = chain_c5(torch, ctx, dev, WP, form=form)
                print(f"[bench] {key}: {out[key]['us_per_forward']} us/forward",
                      file=sys.stderr, flush=True)
            del WP
        del W
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
