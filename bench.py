#!/usr/bin/env python3
"""Benchmark of the MI355X Q4_K linear() path (one JSON line on stdout).

Headline (the benchmark's metric, config 1): the ragged decode batch of 8
sequences x 1 token through the Qwen3.5-9B-shaped MLP with Q4_K weights --
fused gate/up (K=4096 -> N=12288, x2, SiLU(gate)*up into the gate buffer) then
down (K=12288 -> N=4096, residual added in place).  A step is one such MLP
pass; `value` is algorithmic HBM bytes per step / step time (GB/s), with the
inputs resident in HBM and weights rotating over enough copies (> 256 MB
Infinity Cache) that every step streams its weights from HBM.  Steps are
replayed from a HIP graph (launch-bound 5-20 us kernels).

Also reported: config 4 (M=2048 prefill MLP, three Q4_K GEMMs) in TFLOP/s,
the dominant kernels' rooflines from per-launch HIP events, a measured
device-copy bandwidth, and the CPU oracle timed on host cores.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published
FP16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, AMD published
BLOCK_BYTES = 144


def q4k_bytes(n, k):
    return n * (k // 256) * BLOCK_BYTES


def make_q4k(rng, n, k):
    """GGUF block_q4_K bytes: d, dmin = fp16(U(0, 0.01)), uniform scale and quant bytes."""
    import numpy as np
    nb = k // 256
    w = rng.integers(0, 256, size=(n, nb, BLOCK_BYTES), dtype=np.uint8)
    d = rng.uniform(0.0, 0.01, size=(n, nb, 2)).astype(np.float16)
    w[:, :, 0:4] = d.view(np.uint8).reshape(n, nb, 4)
    return w.reshape(-1)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode MLP steps")
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed decode MLP steps before the timed ones (replayed from a graph like them)")
    ap.add_argument("--sets", type=int, default=10, help="rotating weight copies (85 MB each)")
    ap.add_argument("--decode-warmup-ms", type=float, default=300.0,
                    help="untimed decode graph replays (by wall time) after the W warmup steps: a fresh process "
                         "runs its first couple of hundred decode steps about 10 %% slower")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--prefill-warmup-ms", type=float, default=300.0,
                    help="untimed prefill graph replays before the timed ones, and as long again before each config-2/3 "
                         "pass and each typed prefill GEMM shape (the GEMMs run about 15 %% slower for the first tens of "
                         "milliseconds of sustained MFMA work)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-types", action="store_true", help="skip the Q8_0 / Q5_K / IQ4_XS LM-head and the typed prefill GEMM timings")
    ap.add_argument("--part", default="all",
                    choices=["all", "decode", "prefill", "config0", "config2", "config3", "lm_head", "types", "types_prefill", "shard",
                             "neighbours"],
                    help="run one workload alone (for profiling runs that attribute kernel statistics to one configuration)")
    return ap.parse_args()


def timed_graph(graph, replays):
    """Seconds for `replays` replays of a captured graph: HIP events recorded
    on the current stream (where the graph replays) around them."""
    import torch
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3


def graph_kernel_us(fn, count):
    """Average microseconds per call of fn(i) (one kernel launch) over `count`
    calls captured back to back in one graph, as the timed region replays
    them: the launch's duration plus the gap to the next dispatch."""
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(count):
            fn(i)
    timed_graph(g, 2)
    us = timed_graph(g, 3) / (3 * count) * 1e6
    del g
    return us


def kernel_avg_ms(q4k, family):
    launches, total, lo, hi = q4k.profile_query(family)
    return (total / launches if launches else float("nan")), launches


def decode_bench(args, dev):
    import numpy as np
    import torch
    import mtlqwen_amd as q4k

    M, K, N = 8, 4096, 12288
    rng = np.random.default_rng(0x51A70001)
    raw = [torch.from_numpy(make_q4k(rng, n, k)).to(dev) for n, k in ((N, K), (N, K), (K, N))]
    sets = [[q4k.Weight(raw[i], *shape) for i, shape in enumerate(((N, K), (N, K), (K, N)))] for _ in range(args.sets)]
    del raw
    x = (torch.randn(M, K, device=dev, generator=torch.Generator(device=dev).manual_seed(0x51A71001)) * 0.5)
    hidden = torch.randn(M, K, device=dev)
    gate = torch.empty(M, N, device=dev)
    counts = [1] * M

    def step(s):
        G, U, D = sets[s]
        q4k.mlp(x, G, U, D, hidden, gate, M, query_counts=counts)

    # Untimed warmup: one eager step per weight set (first touch), then W
    # steps replayed from a graph of their own.  A fresh process runs its
    # first couple of hundred steps about 10 % slower (measured: a 200-step
    # graph replays at 30.1 us/step first, 27.5 us/step once the device has
    # run that long), so the default W is 200.
    for i in range(len(sets)):
        step(i)
    torch.cuda.synchronize()
    # Then, whatever W is, replays of a 50-step graph until decode_warmup_ms
    # of wall time have passed, so a short --warmup does not time the slow
    # first steps of a fresh process.
    if args.warmup > 0:
        warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(warm):
            for i in range(args.warmup):
                step(i % len(sets))
        warm.replay()
        torch.cuda.synchronize()
        del warm
    if args.decode_warmup_ms > 0:
        warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(warm):
            for i in range(50):
                step(i % len(sets))
        t_end = time.perf_counter() + args.decode_warmup_ms * 1e-3
        while True:
            timed_graph(warm, 1)
            if time.perf_counter() >= t_end:
                break
        del warm

    # Timed region: exactly K steps, replayed from one HIP graph that cycles
    # the weight sets (the graph's first launch is inside the timed region).
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(args.steps):
            step(i % len(sets))
    elapsed = timed_graph(graph, 1)
    ms = elapsed / args.steps * 1e3

    # The same K steps launched eagerly with profiling on: every dispatch
    # carries start/stop events stamped with its own begin/end times
    # (hipExtLaunchKernel), giving per-kernel average durations.
    q4k.profile_enable(True)
    for i in range(args.steps):
        step(i % len(sets))
    torch.cuda.synchronize()
    gated_ms, gated_n = kernel_avg_ms(q4k, q4k.KERNEL_GEMV_GATED)
    down_ms, _ = kernel_avg_ms(q4k, q4k.KERNEL_GEMV)
    _, stage_n = kernel_avg_ms(q4k, q4k.KERNEL_STAGE)
    q4k.profile_enable(False)
    steps = args.steps

    # The decoder's MLP block as the reference runs it (forward.cpp:114-119):
    # x = hidden with the layer's ffn_norm, which the fused gate/up GEMV
    # applies on the way in (no separate rms_norm launch).
    norm_w = torch.full((K,), 0.05, device=dev)
    h_block = torch.randn(M, K, device=dev)
    q4k.profile_enable(True)
    for i in range(args.steps):
        G, U, D = sets[i % len(sets)]
        q4k.mlp(h_block, G, U, D, h_block, gate, M, query_counts=counts, norm_weight=norm_w)
    torch.cuda.synchronize()
    gated_norm_ms, _ = kernel_avg_ms(q4k, q4k.KERNEL_GEMV_GATED)
    aux_ms, aux_n = kernel_avg_ms(q4k, q4k.KERNEL_AUX)
    q4k.profile_enable(False)

    # The two kernels of the step each replayed back to back from a graph, as
    # in the timed region (the eager launches above run each kernel after an
    # idle gap of host launch overhead): these durations set the rooflines.
    gated_graph_us = graph_kernel_us(lambda i: q4k.mlp_gate_up(x, sets[i % len(sets)][0], sets[i % len(sets)][1], M, gate,
                                                               query_counts=counts), args.steps)
    down_graph_us = graph_kernel_us(lambda i: q4k.linear(gate, sets[i % len(sets)][2], M, hidden, auxiliary=hidden,
                                                         query_counts=counts), args.steps)

    wbytes = 2 * q4k_bytes(N, K) + q4k_bytes(K, N)
    act = 4 * (M * K + M * N)  # gate/up: x in, gate buffer out
    act += 4 * (M * N + 2 * M * K)  # down: gate buffer in, residual in + out
    step_bytes = wbytes + act

    # The same step with fp16 activations (the engine's own activation type,
    # quant_linear.metal:119-120): x, hidden and the gate buffer in fp16.
    x16, hidden16, gate16 = (x * 0.2).half(), hidden.half(), gate.half()

    def step16(s):
        G, U, D = sets[s]
        q4k.mlp(x16, G, U, D, hidden16, gate16, M, query_counts=counts)

    for i in range(len(sets)):
        step16(i)
    g16 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g16):
        for i in range(args.steps):
            step16(i % len(sets))
    timed_graph(g16, 3)
    ms16 = timed_graph(g16, 1) / args.steps * 1e3
    q4k.profile_enable(True)
    for i in range(args.steps):
        step16(i % len(sets))
    torch.cuda.synchronize()
    gated16_ms, _ = kernel_avg_ms(q4k, q4k.KERNEL_GEMV_GATED)
    down16_ms, _ = kernel_avg_ms(q4k, q4k.KERNEL_GEMV)
    q4k.profile_enable(False)
    step16_bytes = wbytes + act // 2
    del g16
    gated_bytes = 2 * q4k_bytes(N, K) + 4 * (M * K + M * N)
    down_bytes = q4k_bytes(K, N) + 4 * (M * N + 2 * M * K)
    return {
        "ms_per_step": ms,
        "steps": steps,
        "value": step_bytes / (ms * 1e-3) / 1e9,
        "step_bytes": step_bytes,
        "gated": {"avg_us": gated_graph_us, "event_us": gated_ms * 1e3, "launches": gated_n, "bytes": gated_bytes,
                  "gbs": gated_bytes / (gated_graph_us * 1e-6) / 1e9},
        "down": {"avg_us": down_graph_us, "event_us": down_ms * 1e3, "bytes": down_bytes,
                 "gbs": down_bytes / (down_graph_us * 1e-6) / 1e9},
        "stage_launches": stage_n,
        "gated_norm_us": gated_norm_ms * 1e3,
        "norm_launches": aux_n,
        "weight_sets_mb": len(sets) * wbytes / 1e6,
        "f16": {"ms_per_step": ms16, "gbs": step16_bytes / (ms16 * 1e-3) / 1e9, "step_bytes": step16_bytes,
                "gate_up_us": gated16_ms * 1e3, "down_us": down16_ms * 1e3,
                "gate_up_gbs": (2 * q4k_bytes(N, K) + 2 * (M * K + M * N)) / (gated16_ms * 1e-3) / 1e9},
    }


def config0_bench(dev, sets=32, reps=64):
    """Config 0 on the GPU: one Q4_K linear, M = 1 token, K = N = 4096 (the
    decode GEMV), fp32 activations, weights rotating over 32 copies (302 MB,
    past the 256 MB memory-side cache), launches replayed from a HIP graph;
    plus per-launch times from dispatch-attached events.  The reference
    publishes one kernel time for this shape, on another GPU (an M2 Pro:
    62.08 us, agents/KERNELS.md:54); it is context, not a same-node
    comparison."""
    import numpy as np
    import torch
    import mtlqwen_amd as q4k

    K = N = 4096
    rng = np.random.default_rng(0x51A70000)
    raw = torch.from_numpy(make_q4k(rng, N, K)).to(dev)
    ws = [q4k.Weight(raw, N, K) for _ in range(sets)]
    del raw
    x = torch.randn(1, K, device=dev, generator=torch.Generator(device=dev).manual_seed(0x51A71000))
    y = torch.empty(1, N, device=dev)
    for w in ws:
        q4k.linear(x, w, 1, y, query_counts=[1])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(reps):
            q4k.linear(x, ws[i % sets], 1, y, query_counts=[1])
    timed_graph(graph, 20)
    us = timed_graph(graph, 20) / (20 * reps) * 1e6
    q4k.profile_enable(True)
    for i in range(reps):
        q4k.linear(x, ws[i % sets], 1, y, query_counts=[1])
    torch.cuda.synchronize()
    ev_ms, launches = kernel_avg_ms(q4k, q4k.KERNEL_GEMV)
    _, stage_n = kernel_avg_ms(q4k, q4k.KERNEL_STAGE)
    q4k.profile_enable(False)
    nbytes = q4k_bytes(N, K) + 4 * (K + N)
    return {"workload": "config0: single Q4_K linear M=1, K=N=4096, fp32 x/y (decode GEMV)", "kernel": ws[0].kernel_name(0),
            "us_per_linear": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes,
            "gemv_avg_us": round(ev_ms * 1e3, 3), "launches_per_linear": round((launches + stage_n) / reps, 2),
            "reference_published_us_m2pro": 62.08}


def shard_bench(args, dev):
    """One GPU's share of the config-1 MLP if it were sharded 8 ways (gate/up
    column-parallel over N, down row-parallel over K): the fused gate/up at
    N = 1536 and the down projection at K = 1536, weights rotating over
    args.sets copies, kernel times from dispatch-attached events."""
    import numpy as np
    import torch
    import mtlqwen_amd as q4k

    M, K, N, S = 8, 4096, 12288, 8
    rng = np.random.default_rng(0x51A70008)
    raw = [torch.from_numpy(make_q4k(rng, n, k)).to(dev) for n, k in ((N // S, K), (N // S, K), (K, N // S))]
    sets = [[q4k.Weight(raw[i], *shape) for i, shape in enumerate(((N // S, K), (N // S, K), (K, N // S)))]
            for _ in range(args.sets)]
    x = torch.randn(M, K, device=dev) * 0.5
    gate = torch.empty(M, N // S, device=dev)
    part = torch.empty(M, K, device=dev)
    counts = [1] * M
    for i in range(2 * len(sets)):
        G, U, D = sets[i % len(sets)]
        q4k.mlp_gate_up(x, G, U, M, gate, query_counts=counts)
        q4k.linear(gate, D, M, part, query_counts=counts)
    torch.cuda.synchronize()
    q4k.profile_enable(True)
    for i in range(args.steps):
        G, U, D = sets[i % len(sets)]
        q4k.mlp_gate_up(x, G, U, M, gate, query_counts=counts)
        q4k.linear(gate, D, M, part, query_counts=counts)
    torch.cuda.synchronize()
    gu_ms, _ = kernel_avg_ms(q4k, q4k.KERNEL_GEMV_GATED)
    dn_ms, _ = kernel_avg_ms(q4k, q4k.KERNEL_GEMV)
    q4k.profile_enable(False)
    gu_bytes = 2 * q4k_bytes(N // S, K) + 4 * (M * K + M * N // S)
    dn_bytes = q4k_bytes(K, N // S) + 4 * (M * N // S + M * K)
    return {
        "workload": "config1 MLP, one GPU's share of an 8-way shard: fused gate/up 4096->1536 x2, down 1536->4096 (partial sums)",
        "gate_up_us": round(gu_ms * 1e3, 3), "gate_up_gbs": round(gu_bytes / (gu_ms * 1e-3) / 1e9, 1),
        "down_us": round(dn_ms * 1e3, 3), "down_gbs": round(dn_bytes / (dn_ms * 1e-3) / 1e9, 1),
    }


def neighbours_bench(args, dev):
    """The path's neighbours in a pass, each timed per launch with dispatch-
    attached events: the Q4_K token embedding of 8 decode tokens from a full
    248,320 x 4096 table (quant_linear.metal:572-591), the RMS norm of the 8
    decode rows, and config 3's LM-head rms_norm_gather (8 of 821 rows).
    All three are single round trips of a few KB to a few hundred KB, so
    they are latency-bound; their GB/s are reported for completeness."""
    import torch
    import mtlqwen_amd as q4k

    vocab, k = 248320, 4096
    rb = k // 256 * BLOCK_BYTES
    g = torch.Generator(device=dev).manual_seed(0x51A70005)
    raw = torch.randint(0, 256, (vocab, rb), dtype=torch.uint8, device=dev, generator=g)
    dd = (torch.rand((vocab, k // 256, 2), device=dev, generator=g) * 0.01).half().view(torch.uint8)
    raw.view(vocab, k // 256, BLOCK_BYTES)[:, :, 0:4] = dd.view(vocab, k // 256, 4)
    table = q4k.Weight(raw.reshape(-1), vocab, k)
    del raw, dd
    ids = torch.randint(0, vocab, (8,), dtype=torch.int32, device=dev, generator=g)
    emb = torch.empty((8, k), device=dev)
    w = torch.randn(k, device=dev, generator=g)
    lengths = [512, 37, 1, 1, 200, 5, 1, 64]
    hidden = torch.randn((sum(lengths), k), device=dev, generator=g)
    normed = torch.empty((8, k), device=dev)
    lm_rows = torch.empty((8, k), device=dev)

    def run():
        q4k.embedding(table, ids, emb)
        q4k.rms_norm(emb, w, normed)
        q4k.rms_norm_gather(hidden, w, lm_rows, lengths, [1] * 8)

    for _ in range(10):
        run()
    torch.cuda.synchronize()
    reps = 100
    # All three share one profiling family: time each in a loop of its own.
    out = {}
    for name, fn, nbytes in (
            ("embedding_8_tokens", lambda: q4k.embedding(table, ids, emb), 8 * rb + 8 * k * 4 + 8 * 4),
            ("rms_norm_8_rows", lambda: q4k.rms_norm(emb, w, normed), 2 * 8 * k * 4 + k * 4),
            ("rms_norm_gather_config3", lambda: q4k.rms_norm_gather(hidden, w, lm_rows, lengths, [1] * 8),
             2 * 8 * k * 4 + k * 4)):
        q4k.profile_enable(True)
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        n, tot, lo, _ = q4k.profile_query(q4k.KERNEL_AUX)
        q4k.profile_enable(False)
        avg_us = tot / n * 1e3
        out[name] = {"avg_us": round(avg_us, 3), "min_us": round(lo * 1e3, 3), "bytes": nbytes,
                     "gbs": round(nbytes / (avg_us * 1e-6) / 1e9, 1)}
    return out


def configs_bench(dev, parts=("config2", "config3"), sets=3, warm_ms=300.0):
    """Benchmark configurations 2 and 3, each as one HIP graph of
    its projections (random Q4_K weights as in config 0, seeded fp32
    activations), timed over replays:
      config 2: speculative verify, 8 sequences x 5 tokens = 40 rows, query
        counts 5 (the decode phase, forward.cpp:190): QKV 4096 -> 6144, O
        4096 -> 4096 with the residual, and the config-1 MLP (q4k_mlp);
      config 3: ragged prefill of lengths {512,37,1,1,200,5,1,64} = 821 rows
        (the prefill phase): QKV, O with the residual, gate and up in one
        q4k_mlp_gate_up call (SiLU(gate) * up into the gate buffer, one gated
        GEMM launch), down with the residual, then
        rms_norm_gather of each sequence's last row and the Q4_K LM head
        4096 -> 248,320 on those 8 rows (forward.cpp:72-75, 115-119).
    Reports the time per pass and its algorithmic rate: weight + activation
    bytes for config 2 (HBM-bound), 2 M N K FLOP of the projections for
    config 3 (its prefill GEMMs dominate)."""
    import torch
    import mtlqwen_amd as q4k

    g = torch.Generator(device=dev).manual_seed(0x51A70009)

    def weight(n, k):
        nb = k // 256
        raw = torch.randint(0, 256, (n, nb, 144), dtype=torch.uint8, device=dev, generator=g)
        raw[:, :, 0:4] = (torch.rand((n, nb, 2), device=dev, generator=g) * 0.01).half().view(torch.uint8).view(n, nb, 4)
        return q4k.Weight(raw.reshape(-1), n, k)

    K, F = 4096, 12288
    out = {}
    reps = 20

    def run(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for _ in range(reps):
                fn()
        # Untimed replays for warm_ms of wall time first, as the prefill leg
        # does: kernels of a freshly started stream of work run slower.
        t_end = time.perf_counter() + warm_ms * 1e-3
        while True:
            graph.replay()
            torch.cuda.synchronize()
            if time.perf_counter() >= t_end:
                break
        return timed_graph(graph, 5) / (5 * reps)

    if "config2" in parts:
        # config 2, weights rotating over `sets` copies (118 MB each: more
        # than the 256 MB memory-side cache for sets >= 3)
        wsets = [(weight(6144, K), weight(K, K), weight(F, K), weight(F, K), weight(K, F)) for _ in range(sets)]
        M = 40
        counts = [5] * 8
        x = torch.randn((M, K), device=dev, generator=g)
        hidden = torch.randn((M, K), device=dev, generator=g)
        yq = torch.empty((M, 6144), device=dev)
        gate = torch.empty((M, F), device=dev)
        turn = [0]

        def pass2():
            qkv, o, gw, uw, dw = wsets[turn[0] % len(wsets)]
            turn[0] += 1
            q4k.linear(x, qkv, M, yq, query_counts=counts)
            q4k.linear(x, o, M, hidden, auxiliary=hidden, query_counts=counts)
            q4k.mlp(x, gw, uw, dw, hidden, gate, M, query_counts=counts)

        dt = run(pass2)
        wbytes = (6144 + K + 2 * F) * (K // 256) * 144 + K * (F // 256) * 144
        abytes = 4 * M * (3 * K + 6144 + 2 * K + 2 * F + 2 * K)
        out["config2"] = {"workload": "M=40 (8 x 5 tokens, decode phase): QKV 4096->6144, O 4096->4096 + residual, MLP 4096->12288x2->4096 + residual",
                          "weight_sets": len(wsets), "us_per_pass": round(dt * 1e6, 2), "bytes": wbytes + abytes,
                          "gbs": round((wbytes + abytes) / dt / 1e9, 1), "frac_of_8tbs": round((wbytes + abytes) / dt / 8e12, 3),
                          "kernels": {"qkv": wsets[0][0].kernel_name(0), "gate_up": wsets[0][2].kernel_name(3), "down": wsets[0][4].kernel_name(0)}}
        del wsets
        torch.cuda.empty_cache()
    if "config3" not in parts:
        return out

    # config 3
    qkv, o, gw, uw, dw = weight(6144, K), weight(K, K), weight(F, K), weight(F, K), weight(K, F)
    head = weight(248320, K)
    norm_w = torch.rand(K, device=dev, generator=g) + 0.5
    lengths = [512, 37, 1, 1, 200, 5, 1, 64]
    M = sum(lengths)
    x = torch.randn((M, K), device=dev, generator=g)
    hidden = torch.randn((M, K), device=dev, generator=g)
    yq = torch.empty((M, 6144), device=dev)
    gate = torch.empty((M, F), device=dev)
    lm_rows = torch.empty((8, K), device=dev)
    logits = torch.empty((8, 248320), device=dev)

    def pass3():
        q4k.linear(x, qkv, M, yq, query_counts=lengths)
        q4k.linear(x, o, M, hidden, auxiliary=hidden, query_counts=lengths)
        q4k.mlp_gate_up(x, gw, uw, M, gate, query_counts=lengths)
        q4k.linear(gate, dw, M, hidden, auxiliary=hidden, query_counts=lengths)
        q4k.rms_norm_gather(hidden, norm_w, lm_rows, lengths, [1] * 8)
        q4k.linear(lm_rows, head, 8, logits, query_counts=[8])

    dt = run(pass3)
    flops = 2 * M * K * (6144 + K + 2 * F + F)
    head_flops = 2 * 8 * K * 248320
    out["config3"] = {"workload": "M=821 ragged prefill {512,37,1,1,200,5,1,64}: QKV, O + residual, gate/up (q4k_mlp_gate_up: one gated GEMM launch, SiLU(gate) * up), down + residual, rms_norm_gather, Q4_K LM head 4096->248320 on 8 rows",
                      "us_per_pass": round(dt * 1e6, 2), "projection_flop": flops, "tflops_incl_lm_head": round((flops + head_flops) / dt / 1e12, 1),
                      "kernels": {"prefill": qkv.kernel_name(1), "lm_head": head.kernel_name(2)}}
    return out


def lm_head_bench(dev, ggml_type):
    """The LM head (K = 4096 -> N = 248,320) on 8 gathered rows, as config 3's
    LM-head pass runs it: the decode pack of x, then the persistent GEMV.
    Q4_K (572 MB) is the configuration's own type; Q6_K (834 MB) is what real
    Qwen3.5 GGUF files store as output.weight (quant_linear.metal:644-650).
    Timed per launch with dispatch-attached events (GEMV and pack), and as a
    whole from a graph of both launches."""
    import torch
    import mtlqwen_amd as q4k

    n, k, m = 248320, 4096, 8
    nb = k // 256
    g = torch.Generator(device=dev).manual_seed(0x51A70006 + ggml_type)
    if ggml_type == q4k.GGML_TYPE_Q6_K:
        bb, name = 210, "Q6_K"
        raw = torch.randint(0, 256, (n, nb, bb), dtype=torch.uint8, device=dev, generator=g)
        dd = (torch.rand((n, nb, 1), device=dev, generator=g) * 0.01).half().view(torch.uint8)
        raw[:, :, 208:210] = dd.view(n, nb, 2)
    else:  # Q4_K: d, dmin ~ U(0, 0.01), as in config 0
        bb, name = 144, "Q4_K"
        raw = torch.randint(0, 256, (n, nb, bb), dtype=torch.uint8, device=dev, generator=g)
        dd = (torch.rand((n, nb, 2), device=dev, generator=g) * 0.01).half().view(torch.uint8)
        raw[:, :, 0:4] = dd.view(n, nb, 4)
    W = q4k.Weight(raw.reshape(-1), n, k, ggml_type=ggml_type)
    del raw, dd
    x = torch.randn((m, k), device=dev, generator=g)
    y = torch.empty((m, n), device=dev)
    counts = [1] * m
    for _ in range(5):
        q4k.linear(x, W, m, y, query_counts=counts)
    torch.cuda.synchronize()
    reps = 50
    q4k.profile_enable(True)
    for _ in range(reps):
        q4k.linear(x, W, m, y, query_counts=counts)
    torch.cuda.synchronize()
    ng, tg, lg, _ = q4k.profile_query(q4k.KERNEL_GEMV)
    ns, ts, _, _ = q4k.profile_query(q4k.KERNEL_STAGE)
    q4k.profile_enable(False)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for _ in range(reps):
            q4k.linear(x, W, m, y, query_counts=counts)
    graph.replay()
    torch.cuda.synchronize()
    step_ms = timed_graph(graph, 3) / (3 * reps) * 1e3
    weight_bytes = n * nb * bb
    nbytes = weight_bytes + m * k * 4 + m * n * 4
    gemv_us = tg / ng * 1e3
    return {"shape": f"{name} N={n} K={k} m={m}", "kernel": W.kernel_name(0), "gemv_avg_us": round(gemv_us, 2), "gemv_min_us": round(lg * 1e3, 2),
            "pack_avg_us": round(ts / ns * 1e3, 2), "step_us": round(step_ms * 1e3, 2), "bytes": nbytes,
            "gemv_gbs": round(nbytes / (gemv_us * 1e-6) / 1e9, 1), "gemv_frac_of_8tbs": round(nbytes / (gemv_us * 1e-6) / 8e12, 3),
            "step_gbs": round(nbytes / (step_ms * 1e-3) / 1e9, 1)}


def types_bench(args, dev):
    """The other GGUF types of the linear() surface at the LM-head shape
    (8 rows, K = 4096 -> N = 248,320; persistent GEMV), per launch with
    dispatch-attached events: Q8_0 (1.08 GB), Q5_K (699 MB), IQ4_XS (540 MB)."""
    import torch
    import mtlqwen_amd as q4k

    n, k, m = 248320, 4096, 8
    nb = k // 256
    out = {}
    for name, t in (("q8_0", q4k.GGML_TYPE_Q8_0), ("q5_k", q4k.GGML_TYPE_Q5_K), ("iq4_xs", q4k.GGML_TYPE_IQ4_XS)):
        bb = q4k.q4k_nbytes(1, 256, t)
        g = torch.Generator(device=dev).manual_seed(0x51A70007 + t)
        raw = torch.randint(0, 256, (n * nb * bb,), dtype=torch.uint8, device=dev, generator=g)
        # fp16 scale fields of magnitude below 2^-7 (finite outputs).
        if t == q4k.GGML_TYPE_Q8_0:
            raw.view(n, nb * 8, 34)[:, :, 1] &= 0x1F
        else:
            raw.view(n, nb, bb)[:, :, 1] &= 0x1F
            if t == q4k.GGML_TYPE_Q5_K:
                raw.view(n, nb, bb)[:, :, 3] &= 0x1F
        W = q4k.Weight(raw, n, k, ggml_type=t)
        del raw
        x = torch.randn((m, k), device=dev, generator=g)
        y = torch.empty((m, n), device=dev)
        for _ in range(10):
            q4k.linear(x, W, m, y, query_counts=[1] * m)
        torch.cuda.synchronize()
        q4k.profile_enable(True)
        for _ in range(30):
            q4k.linear(x, W, m, y, query_counts=[1] * m)
        torch.cuda.synchronize()
        ng, tg, _, _ = q4k.profile_query(q4k.KERNEL_GEMV)
        q4k.profile_enable(False)
        us = tg / ng * 1e3
        nbytes = n * nb * bb + m * k * 4 + m * n * 4
        out[name] = {"gemv_avg_us": round(us, 2), "bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac_of_8tbs": round(nbytes / (us * 1e-6) / 8e12, 3)}
        W.close()
        torch.cuda.empty_cache()
    return out


def _random_typed(dev, n, k, t, seed):
    """Random bytes of a GGUF tensor of type t with the fp16 scale fields
    below 2^-7 (finite outputs)."""
    import torch
    import mtlqwen_amd as q4k

    nb = k // 256
    bb = q4k.q4k_nbytes(1, 256, t)
    g = torch.Generator(device=dev).manual_seed(seed)
    raw = torch.randint(0, 256, (n * nb * bb,), dtype=torch.uint8, device=dev, generator=g)
    if t == q4k.GGML_TYPE_Q8_0:
        raw.view(n, nb * 8, 34)[:, :, 1] &= 0x1F
    elif t == q4k.GGML_TYPE_Q6_K:
        raw.view(n, nb, bb)[:, :, 209] &= 0x1F
    else:
        raw.view(n, nb, bb)[:, :, 1] &= 0x1F
        if t == q4k.GGML_TYPE_Q5_K:
            raw.view(n, nb, bb)[:, :, 3] &= 0x1F
    return raw


def types_prefill_bench(dev, warm_ms=300.0):
    """The typed MFMA prefill GEMM at the config-4 shapes (M = 2048; gate
    K = 4096 -> N = 12288 and down K = 12288 -> N = 4096), per launch with
    dispatch-attached events, after warm_ms of untimed back-to-back launches
    of the same call (as the prefill leg warms up)."""
    import torch
    import mtlqwen_amd as q4k

    M = 2048
    out = {}
    for name, t in (("q6_k", q4k.GGML_TYPE_Q6_K), ("q5_k", q4k.GGML_TYPE_Q5_K), ("q8_0", q4k.GGML_TYPE_Q8_0),
                    ("iq4_xs", q4k.GGML_TYPE_IQ4_XS)):
        res = {}
        for shape, (n, k) in (("gate", (12288, 4096)), ("down", (4096, 12288))):
            W = q4k.Weight(_random_typed(dev, n, k, t, 0x51A70040 + t + n), n, k, ggml_type=t)
            x = torch.randn((M, k), device=dev, generator=torch.Generator(device=dev).manual_seed(0x51A70041 + t))
            y = torch.empty((M, n), device=dev)
            t_end = time.perf_counter() + warm_ms * 1e-3
            while True:
                for _ in range(4):
                    q4k.linear(x, W, M, y, query_counts=[M])
                torch.cuda.synchronize()
                if time.perf_counter() >= t_end:
                    break
            q4k.profile_enable(True)
            for _ in range(10):
                q4k.linear(x, W, M, y, query_counts=[M])
            torch.cuda.synchronize()
            gemm_ms, _ = kernel_avg_ms(q4k, q4k.KERNEL_GEMM)
            q4k.profile_enable(False)
            tf = 2.0 * M * n * k / (gemm_ms * 1e-3) / 1e12
            res[shape] = {"gemm_avg_us": round(gemm_ms * 1e3, 1), "tflops": round(tf, 1),
                          "frac_of_peak": round(tf / FP16_DENSE_PEAK_TFLOPS, 4)}
            W.close()
            del x, y
        out[name] = res
        torch.cuda.empty_cache()
    return out


def prefill_bench(args, dev):
    import numpy as np
    import torch
    import mtlqwen_amd as q4k

    M, K, N = 2048, 4096, 12288
    rng = np.random.default_rng(0x51A70004)
    G, U, D = (q4k.Weight(torch.from_numpy(make_q4k(rng, n, k)).to(dev), n, k) for n, k in ((N, K), (N, K), (K, N)))
    x = torch.randn(M, K, device=dev, generator=torch.Generator(device=dev).manual_seed(0x51A71004))
    gate = torch.empty(M, N, device=dev)
    out = torch.empty(M, K, device=dev)
    counts = [M]

    def step():
        q4k.mlp_gate_up(x, G, U, M, gate, query_counts=counts)
        q4k.linear(gate, D, M, out, query_counts=counts)

    step()
    torch.cuda.synchronize()
    # Four steps per graph, as the decode graph holds many: one replay's host
    # launch boundary is then shared by four steps instead of charged to one.
    per_graph = 4
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            step()
    # Untimed warm-up by wall time: in a kernel trace the GEMMs of the first
    # replays run up to 15 % slower than after about 30 ms of back-to-back
    # GEMMs.
    t_end = time.perf_counter() + args.prefill_warmup_ms * 1e-3
    while True:
        timed_graph(graph, 2)
        if time.perf_counter() >= t_end:
            break
    elapsed = timed_graph(graph, args.prefill_steps)
    ms = elapsed / (args.prefill_steps * per_graph) * 1e3
    # Per-kernel durations, each GEMM family timed on its own (eager launches
    # carrying start/stop events): the gated gate/up GEMM (both projections
    # of the step in one launch), then the down GEMM.
    def timed_gemm(fn):
        q4k.profile_enable(True)
        for _ in range(args.prefill_steps):
            fn()
        torch.cuda.synchronize()
        avg, n = kernel_avg_ms(q4k, q4k.KERNEL_GEMM)
        q4k.profile_enable(False)
        return avg, n

    gu_ms, gu_n = timed_gemm(lambda: q4k.mlp_gate_up(x, G, U, M, gate, query_counts=counts))
    dn_ms, dn_n = timed_gemm(lambda: q4k.linear(gate, D, M, out, query_counts=counts))
    flop_gemm = 2.0 * M * N * K

    # The same step with fp16 activations (the engine's activation type).
    x16, gate16, out16 = (x * 0.05).half(), gate.half(), out.half()

    def step16():
        q4k.mlp_gate_up(x16, G, U, M, gate16, query_counts=counts)
        q4k.linear(gate16, D, M, out16, query_counts=counts)

    step16()
    g16 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g16):
        for _ in range(per_graph):
            step16()
    timed_graph(g16, 10)
    ms16 = timed_graph(g16, args.prefill_steps) / (args.prefill_steps * per_graph) * 1e3
    gu16_ms, _ = timed_gemm(lambda: q4k.mlp_gate_up(x16, G, U, M, gate16, query_counts=counts))
    dn16_ms, _ = timed_gemm(lambda: q4k.linear(gate16, D, M, out16, query_counts=counts))
    del g16
    return {
        "ms_per_step": ms,
        "tflops": 3 * flop_gemm / (ms * 1e-3) / 1e12,
        "gated_gemm_avg_us": gu_ms * 1e3,
        "gated_gemm_launches": gu_n,
        "gated_gemm_tflops": 2 * flop_gemm / (gu_ms * 1e-3) / 1e12,
        "down_gemm_avg_us": dn_ms * 1e3,
        "down_gemm_tflops": flop_gemm / (dn_ms * 1e-3) / 1e12,
        "f16": {"ms_per_step": round(ms16, 4), "tflops": round(3 * flop_gemm / (ms16 * 1e-3) / 1e12, 1),
                "gated_gemm_avg_us": round(gu16_ms * 1e3, 2), "gated_gemm_tflops": round(2 * flop_gemm / (gu16_ms * 1e-3) / 1e12, 1),
                "down_gemm_avg_us": round(dn16_ms * 1e3, 2), "down_gemm_tflops": round(flop_gemm / (dn16_ms * 1e-3) / 1e12, 1)},
    }


def profiled_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy-kernel factor),
    or None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


GATE_UP_BYTES = 57147392  # the fused gate/up GEMV's algorithmic bytes at config 1


def read_ceiling(dev, gate_up_us=None):
    """What a plain streaming read of the fused gate/up's byte count reaches on
    this box: 10 rotating buffers of GATE_UP_BYTES (571 MB, past the 256 MB
    memory-side cache), read with the GEMVs' non-temporal 16-byte loads."""
    import torch
    import mtlqwen_amd as q4k
    bufs = [torch.empty(GATE_UP_BYTES, dtype=torch.uint8, device=dev) for _ in range(10)]
    gbs = q4k.read_ceiling(bufs, reps=100)
    del bufs
    out = {"bytes_per_launch": GATE_UP_BYTES, "buffers": 10, "gbs": round(gbs, 1), "frac_of_8tbs": round(gbs / 8000.0, 4),
           "us_per_launch": round(GATE_UP_BYTES / gbs / 1e3, 2)}
    if gate_up_us:
        out["gate_up_gemv_frac_of_this"] = round((GATE_UP_BYTES / gate_up_us / 1e3) / gbs, 4)
    return out


def copy_ceiling(dev):
    import torch
    n = 1 << 28  # 1 GiB of fp32
    a = torch.empty(n, device=dev)
    b = torch.empty(n, device=dev)
    b.copy_(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    reps = 10
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    return 2 * 4 * n * reps / (time.perf_counter() - t0) / 1e9


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """Host threads for the CPU baseline: every core this process may run on,
    up to the share the GPU box allots one GPU (OMP_NUM_THREADS there: 16),
    so the baseline does not oversubscribe the cores of other jobs."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(avail, share) if share > 0 else avail)


def cpu_baseline(args):
    """The C oracle (a port of the reference's arithmetic; the reference itself
    is Metal-only) on the config-1 MLP, on every host core allotted to this
    process (cpu_threads)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from q4k_ref import Oracle

    oracle = Oracle()
    M, K, N = 8, 4096, 12288
    rng = np.random.default_rng(0x51A70001)
    wg, wu, wd = make_q4k(rng, N, K), make_q4k(rng, N, K), make_q4k(rng, K, N)
    x = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
    hidden = rng.standard_normal((M, K)).astype(np.float32)
    threads = cpu_threads()
    iters, t0 = 0, time.perf_counter()
    while True:
        g = oracle.mlp_gate_up(x, wg, wu, N, K, threads=threads)
        oracle.linear(g, wd, K, N, aux=hidden, post=1, threads=threads)
        iters += 1
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    dt = (time.perf_counter() - t0) / iters
    step_bytes = 2 * q4k_bytes(N, K) + q4k_bytes(K, N) + 4 * (M * K + M * N) + 4 * (M * N + 2 * M * K)

    def timed(fn, budget):
        n, t1 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            if time.perf_counter() - t1 >= budget:
                return (time.perf_counter() - t1) / n, n

    # The other headline configs, on bounded samples (a quarter of the budget each).
    w0 = make_q4k(rng, 4096, 4096)
    x0 = rng.standard_normal((1, 4096)).astype(np.float32)
    dt0, n0 = timed(lambda: oracle.linear(x0, w0, 4096, 4096, threads=threads), args.cpu_seconds / 4)
    rows4 = 16  # config 4 (M=2048) is timed on 16 of its token rows and reported per token
    x4 = rng.standard_normal((rows4, K)).astype(np.float32)

    def mlp4():
        g4 = oracle.mlp_gate_up(x4, wg, wu, N, K, threads=threads)
        oracle.linear(g4, wd, K, N, threads=threads)

    dt4, n4 = timed(mlp4, args.cpu_seconds / 4)
    flop_tok = 3 * 2.0 * N * K
    return {"value": step_bytes / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "cores_note": "threads = the cores allotted to this process (OMP_NUM_THREADS share of the GPU box, within its CPU affinity)",
            "sample": f"{iters} config-1 MLP steps (M=8, gate/up 4096->12288 x2 + down 12288->4096) "
                      f"in {dt * iters:.1f} s, {dt * 1e3:.1f} ms/step",
            "configs": {
                "config0_gbs": round((q4k_bytes(4096, 4096) + 4 * (4096 + 4096)) / dt0 / 1e9, 3),
                "config0_sample": f"{n0} single linears M=1 K=N=4096, {dt0 * 1e3:.2f} ms each",
                "config4_ms_per_token": round(dt4 / rows4 * 1e3, 3),
                "config4_tflops": round(rows4 * flop_tok / dt4 / 1e12, 4),
                "config4_sample": f"{n4} MLP passes over {rows4} token rows (gate/up + down), {dt4 * 1e3:.1f} ms each",
            }}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the Q4_K path has no multi-GPU sharding "
                                   "(gate/up would shard column-parallel over N, down row-parallel over K with one all-reduce); run with --gpus 1"}))
        sys.exit(2)
    import torch
    import mtlqwen_amd  # fails loudly if libq4k.so is missing
    dev = torch.device("cuda:0")

    want = (lambda p: args.part in ("all", p))
    if args.part != "all" and args.part != "decode":
        # one workload alone (profiling runs); printed as its own JSON line
        res = {"part": args.part}
        if args.part == "prefill":
            res["prefill"] = prefill_bench(args, dev)
        elif args.part == "config0":
            res["config0"] = config0_bench(dev)
        elif args.part in ("config2", "config3"):
            res.update(configs_bench(dev, parts=(args.part,), sets=args.sets if args.part == "config2" else 1, warm_ms=args.prefill_warmup_ms))
        elif args.part == "lm_head":
            res["q4k_lm_head"], res["q6k_lm_head"] = lm_head_bench(dev, 12), lm_head_bench(dev, 14)
        elif args.part == "types":
            res["types_lm_head"] = types_bench(args, dev)
        elif args.part == "types_prefill":
            res["types_prefill"] = types_prefill_bench(dev, args.prefill_warmup_ms)
        elif args.part == "shard":
            res["shard_1of8"] = shard_bench(args, dev)
        elif args.part == "neighbours":
            res["neighbours"] = neighbours_bench(args, dev)
        # the 1 GiB device copy that calibrates the FETCH_SIZE / WRITE_SIZE counters
        res["copy_ceiling_gbs"] = round(copy_ceiling(dev), 1)
        print(json.dumps(res), flush=True)
        return

    dec = decode_bench(args, dev)
    cfg0 = config0_bench(dev) if want("config0") else None
    pre = None if args.no_prefill or not want("prefill") else prefill_bench(args, dev)
    shard = shard_bench(args, dev) if want("shard") else None
    neighbours = neighbours_bench(args, dev) if want("neighbours") else None
    cfgs = configs_bench(dev, sets=min(args.sets, 3), warm_ms=args.prefill_warmup_ms) if want("config2") else None
    q4k_head = lm_head_bench(dev, 12) if want("lm_head") else None
    q6k = lm_head_bench(dev, 14) if want("lm_head") else None
    types = None if args.no_types or not want("types") else types_bench(args, dev)
    types_pre = None if args.no_types or args.no_prefill or not want("types_prefill") else types_prefill_bench(dev, args.prefill_warmup_ms)
    copy_gbs = copy_ceiling(dev)
    mfma_tf = mtlqwen_amd.mfma_ceiling(0)
    read_ceil = read_ceiling(dev, dec["gated"]["avg_us"] if "avg_us" in dec.get("gated", {}) else None)
    cpu = None if args.no_cpu else cpu_baseline(args)

    g = dec["gated"]
    line = {
        "metric": "Q4_K linear: HBM GB/s at M=8 decode; TFLOP/s at M=2048 prefill",
        "value": round(dec["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded Q4_K weights per the config-0 recipe, N(0,1)*0.5 activations)",
        "config": {
            "workload": "config1: ragged decode M=8 (8 seqs x 1 token), Q4_K MLP: fused gate/up 4096->12288 x2 "
                        "+ down 12288->4096 with in-place residual (q4k_mlp: two launches); HIP-graph replay",
            "m": 8, "k": 4096, "n": 12288, "weight_sets": len(range(args.sets)),
            "weight_bytes_per_step": dec["step_bytes"],
        },
        "roofline": {
            "kernel": "q4k_gemv_gate_up_kernel (fused gate/up packing x in registers, M=8, K=4096, N=12288)",
            "bound": "hbm",
            "achieved": round(g["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic("gemv_gate_up_m8_traffic.txt"),
            "avg_us": round(g["avg_us"], 3),
            "avg_us_from": "graph of the kernel's launches replayed back to back (HIP events), as in the timed region",
            "eager_event_us": round(g["event_us"], 3),
            "algorithmic_bytes": g["bytes"],
        },
        "kernels": {
            "down_gemv_us": round(dec["down"]["avg_us"], 3),
            "down_gemv_gbs": round(dec["down"]["gbs"], 1),
            # activation staging launches per step (none: both GEMVs pack x themselves)
            "stage_launches_per_step": dec["stage_launches"] / dec["steps"],
            # the same gate/up launch with the layer's ffn_norm applied inside it (x = hidden);
            # no separate RMS-norm launch runs (norm_launches_per_step)
            "gate_up_gemv_with_ffn_norm_us": round(dec["gated_norm_us"], 3),
            "norm_launches_per_step": dec["norm_launches"] / dec["steps"],
        },
        # config 1 with fp16 activations (x, hidden, gate buffer): the engine's own activation type
        "f16_activations": {"ms_per_step": round(dec["f16"]["ms_per_step"], 5), "gbs": round(dec["f16"]["gbs"], 1),
                            "step_bytes": dec["f16"]["step_bytes"], "gate_up_us": round(dec["f16"]["gate_up_us"], 3),
                            "gate_up_gbs": round(dec["f16"]["gate_up_gbs"], 1), "down_us": round(dec["f16"]["down_us"], 3)},
        "decode_warmup_ms": args.decode_warmup_ms,
        "config0": cfg0,
        "shard_1of8": shard,
        "neighbours": neighbours,
        "configs_2_3": cfgs,
        "q4k_lm_head": q4k_head,
        "q6k_lm_head": q6k,
        "types_lm_head": types,
        "types_prefill": types_pre,
        "copy_ceiling_gbs": round(copy_gbs, 1),
        "hbm_read_ceiling": read_ceil,
        "mfma_ceiling_tflops": round(mfma_tf, 1),
        "cpu_baseline": cpu,
    }
    if pre:
        line["prefill"] = {
            "workload": "config4: M=2048 Q4_K MLP on MFMA GEMM: gate and up in one gated GEMM launch (SiLU(gate) * up into the gate buffer), then down",
            "value": round(pre["tflops"], 2),
            "unit": "TFLOP/s",
            "ms_per_step": round(pre["ms_per_step"], 4),
            "roofline": {
                "kernel": "typed_gemm_kernel<Six<TgQ4K>,float,true> (gated gate/up GEMM, six B column tiles per wave, M=2048, K=4096, N=12288 x2: 412.32 GFLOP per launch)",
                "bound": "mfma",
                "achieved": round(pre["gated_gemm_tflops"], 1),
                "peak": FP16_DENSE_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(pre["gated_gemm_tflops"] / FP16_DENSE_PEAK_TFLOPS, 4),
                "traffic": profiled_traffic("gemm2_config4_traffic.txt"),
                "avg_us": round(pre["gated_gemm_avg_us"], 2),
            },
            "down_gemm": {"kernel": "q4k_gemm2_kernel<float,false,false> (K=12288 -> N=4096, 206.16 GFLOP)",
                          "avg_us": round(pre["down_gemm_avg_us"], 2), "tflops": round(pre["down_gemm_tflops"], 1),
                          "frac": round(pre["down_gemm_tflops"] / FP16_DENSE_PEAK_TFLOPS, 4)},
            # the same step with fp16 activations (x scaled by 0.05 to stay in fp16 range)
            "f16_activations": pre["f16"],
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
