#!/usr/bin/env python3
"""Benchmark of the GGUF quantized matrix-vector hot path on one MI355X.

Default workload: Q4_K matvec 4096 -> 14336 at batch 1 with fp16 activations,
the configuration the headline metric is quoted on. A step is one matvec
launch over one batch of synthetic input; the weights rotate over enough
distinct device copies (>= 2x the 256 MB Infinity Cache) that every step reads
its weights from HBM.

Two timed passes over the same K steps:
  * whole job: the K launches captured in one HIP graph, timed with events
    around the graph launch -> ms_per_step and `value` (GB/s of algorithmic
    bytes, inputs resident in HBM);
  * kernel: each launch's dispatch records its own start/stop events
    (rqmv_matvec_timed) -> the average kernel duration behind
    roofline.achieved, comparable with a rocprofv3 kernel trace.
The CPU baseline times the oracle's restatement of recipe's CPU path (fp32,
exact per-weight decode, sequential fma per block, all rows split over
threads) on a bounded sample of the same workload.

Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "recipe-dev_amd")]

import numpy as np  # noqa: E402

METRIC = "Q4_K matvec effective HBM GB/s (% of peak) at batch 1; decode tok/s"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 * 2 ** 20

WORKLOADS = {
    "q4_k_up": ("q4_k", 14336, 4096, "f16", "Q4_K matvec 4096->14336 batch 1 (FFN up/gate)"),
    "q4_k_down": ("q4_k", 4096, 14336, "f16", "Q4_K matvec 14336->4096 batch 1 (FFN down)"),
    "q4_k_4096": ("q4_k", 4096, 4096, "f16", "Q4_K matvec 4096->4096 batch 1 (attention output)"),
    "q4_0_up": ("q4_0", 14336, 4096, "f16", "Q4_0 matvec 4096->14336 batch 1"),
    "q4_0_down": ("q4_0", 4096, 14336, "f16", "Q4_0 matvec 14336->4096 batch 1"),
    "q8_0_4096": ("q8_0", 4096, 4096, "f32", "Q8_0 matvec 4096x4096, fp32 activations"),
    "q6_k_25600": ("q6_k", 25600, 5120, "f16", "Q6_K matvec 5120->25600, M activation rows"),
    "q8_0_5120": ("q8_0", 5120, 5120, "f16", "Q8_0 matvec 5120->5120, M activation rows"),
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _profile_entry(name, key):
    """One workload's entry of a measured-counter file under profiles/, if recorded."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    try:
        return json.load(open(path)).get(key)
    except (OSError, ValueError):
        return None


def traffic_from_profiles(workload, m):
    """HBM bytes per launch measured by rocprofv3 counters, if recorded."""
    return _profile_entry("traffic.json", f"{workload}_m{m}")


def rocprof_roofline(workload, m, alg_bytes):
    """The dominant kernel's mean duration in a committed rocprofv3 kernel
    trace of the same bench command, and the roofline fraction it gives: the
    profiler's dispatch timestamps, beside the live event timing."""
    e = _profile_entry("kernel_time.json", f"{workload}_m{m}")
    if not e:
        return None
    gbs = alg_bytes / (e["mean_us"] * 1e-6) / 1e9
    return {"kernel": e["kernel"], "mean_us": e["mean_us"], "achieved": round(gbs, 2),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "source": e["source"]}


def host_cpu():
    """Threads the CPU baseline runs on, and the host it ran on. recipe's CPU
    backend runs one worker per host core (cpu-worker-threads = 0, Cargo.toml:52;
    recipe.rs:28613-28616): every core in this process's affinity mask, capped
    by OMP_NUM_THREADS where the host grants a job a share of its cores."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    threads = affinity
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        threads = min(threads, int(share))
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return threads, {"nproc": os.cpu_count(), "affinity": affinity, "omp_num_threads": share or None,
                     "cpu_model": model}


def stream_copy(achieved_gbs, nbytes=1 << 30, reps=20):
    """The device's STREAM copy rate measured in the same process: a
    stream-ordered device-to-device copy of nbytes (the HIP runtime's copy
    kernel), bytes read plus bytes written over the mean of `reps` copies; and
    the workload's achieved rate as a fraction of it (the second roofline
    fraction beside the 8 TB/s vendor peak)."""
    import rqmv

    src, dst, st = rqmv.DeviceBuffer(nbytes), rqmv.DeviceBuffer(nbytes), rqmv.Stream()
    src.fill_zero()
    for _ in range(3):
        dst.copy_from(src, nbytes, st)
    e0, e1 = rqmv.Event(), rqmv.Event()
    e0.record(st)
    for _ in range(reps):
        dst.copy_from(src, nbytes, st)
    e1.record(st)
    e1.synchronize()
    gbs = 2 * nbytes * reps / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    for o in (src, dst, st, e0, e1):
        o.close()
    log(f"bench: device copy {gbs:.0f} GB/s (read + write)")
    return {"value": round(gbs, 1), "unit": "GB/s", "bytes_per_copy": 2 * nbytes,
            "method": "hipMemcpyAsync device to device of 1 GiB, bytes read + written",
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "workload_frac_of_copy": round(achieved_gbs / gbs, 4)}


def cpu_baseline(fmt, rows, cols, x32, seconds, weights_bytes, alg_bytes):
    import oracle

    cores, host = host_cpu()
    # the same matvec, repeated over the full weight for ~`seconds`
    runs, t0 = 0, time.perf_counter()
    while True:
        oracle.matvec_recipe_fast(fmt, weights_bytes, rows, cols, x32, threads=cores)
        runs += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / runs
    return {"value": round(alg_bytes / per / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port", **host,
            "sample": f"{runs} full {fmt} {cols}->{rows} matvecs (M={x32.shape[0]}) in {el:.1f} s, "
                      f"{per * 1e3:.2f} ms each: recipe's fp32 float path (exact fp32 weights, fp32 fma chain per "
                      f"block, eight rows per SIMD lane group) restated in C, {cores} threads"}


def copy_calibration(mb, steps):
    """A plain copy of known size, so that rocprofv3's FETCH_SIZE / WRITE_SIZE
    per dispatch can be converted to bytes (factor = known bytes / counter)."""
    import torch

    n = mb * 2 ** 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    src.fill_(7)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n, "steps": steps}), flush=True)


def moe_bench(args):
    """The gguf_moe decode step at batch 1: d_model 2048, 256 experts of hidden
    512 in Q4_K, top-8 softmax routing with renormalisation, fp16 router
    2048x256, and a sigmoid-gated shared expert of the same shape. A step is
    one rqmv_moe call (router, top-k, gate/up, down). Two copies of every
    weight (about 0.9 GB) and 16 different tokens rotate, so the selected
    experts change from step to step and the banks do not stay in the
    Infinity Cache."""
    import rqmv
    from rqmv import synth

    d, E, top, H = 2048, 256, 8, 512
    rqmv.init(0)
    log(f"bench: moe_c4 d={d} E={E} top={top} hidden={H} steps={args.steps}")
    sets, hosts = [], []
    for c in range(2):
        seed = 17 + 100 * c
        router = synth.f16_weights(E, d, 0.02, seed=seed, tag="router")
        gate = synth.q4_k(E * H, d, seed=seed + 1, tag="gate")
        up = synth.q4_k(E * H, d, seed=seed + 2, tag="up")
        down = synth.q4_k(E * d, H, seed=seed + 3, tag="down")
        sg = synth.f16_weights(1, d, 0.02, seed=seed + 4, tag="sg")
        gs, us = synth.q4_k(H, d, seed=seed + 5, tag="gs"), synth.q4_k(H, d, seed=seed + 6, tag="us")
        ds = synth.q4_k(d, H, seed=seed + 7, tag="ds")
        moe = rqmv.Moe(rqmv.Weight("f16", E, d, router), rqmv.Weight("q4_k", H, d, gate, experts=E),
                       rqmv.Weight("q4_k", H, d, up, experts=E), rqmv.Weight("q4_k", d, H, down, experts=E), top,
                       scoring=rqmv.SCORE_SOFTMAX, renormalize=True, shared_gate_inp=rqmv.Weight("f16", 1, d, sg),
                       gate_sh=rqmv.Weight("q4_k", H, d, gs), up_sh=rqmv.Weight("q4_k", H, d, us),
                       down_sh=rqmv.Weight("q4_k", d, H, ds))
        sets.append(moe)
        hosts.append((router, gate, up, down, sg, gs, us, ds))
    m = args.m
    tokens = [synth.activations_f16(d, seed=1000 + t) for t in range(16)]
    # step i takes positions i*m .. i*m+m-1 of the 16 tokens, cyclically
    batches = [np.stack([tokens[(i * m + j) % 16] for j in range(m)]) for i in range(16)]
    xbs = [rqmv.DeviceBuffer.from_array(b) for b in batches]
    yb = rqmv.DeviceBuffer(4 * d * m)
    rb = rqmv.DeviceBuffer(4 * E * m)
    stream = rqmv.Stream()
    ws = sets[0].batch_workspace(m)
    expert_bytes = 3 * (H * d // 256 * 144)
    # bytes a step must read: the router, every expert some position of the
    # batch selected (once), the shared expert, x and y
    distinct = []
    for i in range(16):
        sets[0].run_batch(xbs[i], rqmv.DTYPE_F16, m, d, yb, d, rb, ws, stream)
        stream.synchronize()
        distinct.append(int(np.count_nonzero(rb.download(np.float32).reshape(m, E).any(axis=0))))
    alg_bytes = E * d * 2 + d * 2 + expert_bytes * (float(np.mean(distinct)) + 1) + m * (d * 2 + d * 4)
    # flops of a step: per position the router and the shared gate, and gate,
    # up and down of the top-k routed experts and the shared one
    flops = float(m) * (2 * E * d + 2 * d + (top + 1) * 6 * H * d)

    rel = None
    if not args.no_check:
        import oracle

        sets[0].run_batch(xbs[0], rqmv.DTYPE_F16, m, d, yb, d, None, ws, stream)
        stream.synchronize()
        y = yb.download(np.float32)[-d:]  # the batch's last position
        router, gate, up, down, sg, gs, us, ds = hosts[0]
        x64 = synth.fp16_to_f32(batches[0][-1]).astype(np.float64)
        ref, _ = oracle.moe_f64("q4_k", d, E, top, H, router.view(np.uint16), gate, up, down, x64, scoring=0,
                                renormalize=True, hidden_shared=H, shared_gate_bits=sg.view(np.uint16), gate_sh=gs,
                                up_sh=us, down_sh=ds)
        rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
        log(f"bench: parity rel-L2 {rel:.3e}")
        if not rel <= 1e-3:
            log("bench: parity check failed")
            sys.exit(1)

    def enqueue_steps(count):
        for i in range(count):
            if m == 1:
                sets[i % 2].run(xbs[i % 16], rqmv.DTYPE_F16, yb, stream=stream)
            else:
                sets[i % 2].run_batch(xbs[i % 16], rqmv.DTYPE_F16, m, d, yb, d, None, ws, stream)

    graph = rqmv.Graph(stream, lambda: enqueue_steps(args.steps))
    graph.launch(stream)
    stream.synchronize()
    e0, e1 = rqmv.Event(), rqmv.Event()
    e0.record(stream)
    graph.launch(stream)
    e1.record(stream)
    e1.synchronize()
    ms_per_step = e0.elapsed_ms(e1) / args.steps
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"bench: graph {args.steps} steps -> {ms_per_step * 1e3:.2f} us/step, {m / ms_per_step * 1e3:.0f} positions/s")
    out = {
        "metric": "gguf_moe decode step effective HBM GB/s at batch 1" if m == 1 else
                  f"gguf_moe block effective HBM GB/s over a batch of {m} positions",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "gguf_moe decode step: d_model 2048, 256 Q4_K experts of hidden 512, top-8 softmax "
                               "renormalised, fp16 router, sigmoid-gated shared expert", "bytes_per_step": alg_bytes,
                   "flops_per_step": flops,
                   "positions": m, "distinct_experts_per_step": float(np.mean(distinct)),
                   "positions_per_s": round(m / ms_per_step * 1e3, 1),
                   "launches_per_step": 3, "weight_sets": 2, "tokens": 16, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles("moe_c4", m),
                     "note": "whole step (three launches) from the graph replay; traffic sums the three kernels"},
        "stream_copy": stream_copy(value),
        "gflops": round(flops / (ms_per_step * 1e-3) / 1e9, 1),
        "parity_rel_l2": rel,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = moe_cpu_baseline(hosts[0], tokens, d, E, top, H, alg_bytes, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    graph.close()


def moe_cpu_baseline(host, tokens, d, E, top, H, alg_bytes, seconds):
    """recipe's CPU path for the gguf_moe step at one position: the fp16
    router in fp32, top-k, then each selected expert's and the shared
    expert's gate and up rows, SiLU-GLU and down rows on the fp32 float path
    (oracle.matvec_recipe_fast), experts and their row halves spread over the
    CPU share's threads; one step checked against the f64 oracle first."""
    import oracle
    from concurrent.futures import ThreadPoolExecutor

    from rqmv import synth

    cores, hostinfo = host_cpu()
    router, gate, up, down, sg, gs, us, ds = host
    rw = synth.fp16_to_f32(router.view(np.uint16)).reshape(E, d)
    sgw = synth.fp16_to_f32(sg.view(np.uint16)).reshape(d)
    eb_up, eb_down = H * d // 256 * 144, d * H // 256 * 144
    split = max(1, cores // (top + 1))

    def silu(v):
        return v * (np.float32(0.5) * (np.tanh(np.float32(0.5) * v) + np.float32(1.0)))

    def rows_of(n):
        return [(n * c // split, n * (c + 1) // split) for c in range(split)]

    def step(pool, x):
        logits = (rw @ x).astype(np.float64)
        wts = oracle.topk(logits, top, scoring=0, renormalize=True)
        chosen = [int(e) for e in np.nonzero(wts)[0]]
        banks = [(gate[e * eb_up:(e + 1) * eb_up], up[e * eb_up:(e + 1) * eb_up], down[e * eb_down:(e + 1) * eb_down])
                 for e in chosen] + [(gs, us, ds)]
        hidden = [np.empty(H, np.float32) for _ in banks]

        def glu(j, r0, r1):
            g, u, _ = banks[j]
            rb = d // 256 * 144
            a = oracle.matvec_recipe_fast("q4_k", g[r0 * rb:r1 * rb], r1 - r0, d, x)[0]
            b = oracle.matvec_recipe_fast("q4_k", u[r0 * rb:r1 * rb], r1 - r0, d, x)[0]
            hidden[j][r0:r1] = silu(a) * b

        list(pool.map(lambda t: glu(*t), [(j, r0, r1) for j in range(len(banks)) for r0, r1 in rows_of(H)]))
        outs = [np.empty(d, np.float32) for _ in banks]

        def dn(j, r0, r1):
            rb = H // 256 * 144
            outs[j][r0:r1] = oracle.matvec_recipe_fast("q4_k", banks[j][2][r0 * rb:r1 * rb], r1 - r0, H, hidden[j])[0]

        list(pool.map(lambda t: dn(*t), [(j, r0, r1) for j in range(len(banks)) for r0, r1 in rows_of(d)]))
        y = np.zeros(d, np.float32)
        for j, e in enumerate(chosen):
            y += np.float32(wts[e]) * outs[j]
        gate_w = np.float32(1.0) / (np.float32(1.0) + np.exp(-np.float32(sgw @ x)))
        return y + gate_w * outs[-1]

    with ThreadPoolExecutor(cores) as pool:
        x0 = synth.fp16_to_f32(tokens[0])
        got = step(pool, x0)
        ref, _ = oracle.moe_f64("q4_k", d, E, top, H, router.view(np.uint16), gate, up, down, x0.astype(np.float64),
                                scoring=0, renormalize=True, hidden_shared=H, shared_gate_bits=sg.view(np.uint16),
                                gate_sh=gs, up_sh=us, down_sh=ds)
        rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
        runs, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            step(pool, synth.fp16_to_f32(tokens[runs % 16]))
            runs += 1
        el = time.perf_counter() - t0
    return {"value": round(alg_bytes * runs / el / 1e9, 3), "unit": "GB/s", "cores": min(cores, (top + 1) * split),
            "kind": "port", **hostinfo,
            "sample": f"{runs} moe steps in {el:.1f} s ({el / runs * 1e3:.2f} ms each): fp32 router, top-8, the "
                      f"9 experts' products on recipe's fp32 float path, {(top + 1) * split} tasks per phase over "
                      f"{cores} threads; rel-L2 {rel:.1e} against the f64 oracle"}


def decode_bench(args):
    """Single-token decode of a random-init 32-layer decoder: d 4096, 32 query
    and 8 kv heads of 128, NeoX rotary (base 500000), SiLU-GLU of 14336,
    RMSNorm eps 1e-5, every projection Q4_K (fused QKV and gate|up), the
    128256-token head Q8_0, an fp16 KV cache prefilled N(0, 1) to 4096
    positions. A step is one token: embedding row, 32 layers, final norm,
    head, argmax, position advance, replayed from one captured HIP graph with
    the token and position in device memory (greedy decoding). Every layer
    holds its own weight bytes (about 5 GB streamed per token), so nothing is
    served from the Infinity Cache."""
    import rqmv
    from rqmv import synth
    from rqmv.decode import DecodeModel, DecoderShape

    shape = DecoderShape()
    ctx = 4096
    max_ctx = ctx + args.warmup + args.steps + 8
    rqmv.init(0)
    log(f"bench: decode_c5 layers={shape.layers} d={shape.d} ctx={ctx} steps={args.steps} warmup={args.warmup}")
    t0 = time.perf_counter()
    D = synth.DecoderSynth(shape)
    model = DecodeModel(shape, max_ctx, D.embed(), D.out_norm(), D.head())
    layer0 = None
    for i in range(shape.layers):
        t = D.layer(i)
        model.set_layer(i, t)
        model.set_cache(i, *D.cache(i, ctx))
        if i == 0:
            layer0 = t
    rqmv.synchronize()
    log(f"bench: model built in {time.perf_counter() - t0:.1f} s")
    stream = rqmv.Stream()
    model.set_position(1, ctx)
    model.step(stream)  # one eager step first
    stream.synchronize()
    logits = model.read_logits()
    tok = model.read_token()
    ok = bool(np.isfinite(logits).all()) and tok == int(np.argmax(logits)) and model.read_position() == ctx + 1
    log(f"bench: eager step token {tok} finite={bool(np.isfinite(logits).all())} consistent={ok}")
    if not ok and not args.no_check:
        log("bench: decode step check failed")
        sys.exit(1)
    graph = model.capture(stream)
    model.replay(graph, stream, args.warmup)
    stream.synchronize()
    pos0 = model.read_position()
    e0, e1 = rqmv.Event(), rqmv.Event()
    e0.record(stream)
    model.replay(graph, stream, args.steps)
    e1.record(stream)
    e1.synchronize()
    total_ms = e0.elapsed_ms(e1)
    ms_per_step = total_ms / args.steps
    tok_s = 1000.0 / ms_per_step
    assert model.read_position() == pos0 + args.steps
    # bytes one token streams: every projection and the head as stored, the
    # KV cache up to the position (keys and values, fp16), embedding row,
    # norm scales, activations in and out of each projection
    s = shape
    mean_len = pos0 + (args.steps + 1) / 2.0
    kv_bytes = s.layers * 2 * s.kv_heads * mean_len * s.head_dim * 2
    small = s.d * 4 + (2 * s.layers + 1) * s.d * 4
    bytes_per_token = model.weight_bytes() + kv_bytes + small
    achieved = bytes_per_token * tok_s / 1e9
    # flops of a token: every projection and the head (2 per weight), and the
    # attention's scores and weighted sum over the context
    qkv_rows = (s.q_heads + 2 * s.kv_heads) * s.head_dim
    per_layer = s.d * qkv_rows + s.q_heads * s.head_dim * s.d + 2 * s.ffn * s.d + s.d * s.ffn
    flops_per_token = 2.0 * (s.layers * per_layer + s.vocab * s.d) + s.layers * 4.0 * s.q_heads * mean_len * s.head_dim
    log(f"bench: {args.steps} steps {total_ms:.2f} ms -> {ms_per_step * 1e3:.1f} us/token, {tok_s:.1f} tok/s, "
        f"{achieved:.0f} GB/s over {bytes_per_token / 1e9:.3f} GB/token")
    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "single-token decode, random-init 32-layer decoder: d 4096, 32/8 heads of 128, "
                               "NeoX rotary base 500000, SiLU-GLU 14336, RMSNorm 1e-5, Q4_K projections, "
                               "Q8_0 head 128256, fp16 KV cache prefilled to 4096",
                   "bytes_per_token": int(bytes_per_token), "flops_per_token": flops_per_token,
                   "positions": [pos0, pos0 + args.steps - 1],
                   "launches_per_token": 1 + 6 * s.layers + 4, "activations": "f32", "kv_cache": "f16",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles("decode_c5", 1),
                     "note": "whole token (every launch of the step) from graph replays; traffic sums every "
                             "kernel of one token"},
        "stream_copy": stream_copy(achieved),
        "gflops": round(flops_per_token * tok_s / 1e9, 1),
    }
    if not args.no_cpu:
        import oracle

        cores, hostinfo = host_cpu()
        # recipe's CPU float path on layer 0's four projections, timed per layer
        # and scaled to 32 layers, plus the head, plus f64 attention over one
        # layer's cache scaled to 32 layers
        xs = {"qkv": s.d, "o": s.d, "gate": s.d, "up": s.d, "down": s.ffn}
        rows = {"qkv": s.qkv_rows, "o": s.d, "gate": s.ffn, "up": s.ffn, "down": s.d}
        rng = np.random.default_rng(0)
        t0 = time.perf_counter()
        runs = 0
        while time.perf_counter() - t0 < args.cpu_seconds * 0.6:
            for k in ("qkv", "o", "gate", "up", "down"):
                oracle.matvec_recipe_fast(s.proj_fmt, getattr(layer0, k), rows[k], xs[k],
                                          rng.standard_normal(xs[k]).astype(np.float32), threads=cores)
            runs += 1
        layer_s = (time.perf_counter() - t0) / runs
        head = D.head()
        t0 = time.perf_counter()
        oracle.matvec_recipe_fast(s.head_fmt, head, s.vocab, s.d, rng.standard_normal(s.d).astype(np.float32),
                                  threads=cores)
        head_s = time.perf_counter() - t0
        from oracle import decode as oref
        kc, vc = D.cache(0, ctx)
        q = rng.standard_normal((s.q_heads, s.head_dim))
        t0 = time.perf_counter()
        oref.attention(q, kc.view(np.float16).astype(np.float32), vc.view(np.float16).astype(np.float32), ctx)
        attn_s = time.perf_counter() - t0
        token_s = s.layers * (layer_s + attn_s) + head_s
        out["cpu_baseline"] = {
            "value": round(1.0 / token_s, 4), "unit": "tok/s", "cores": cores, "kind": "port", **hostinfo,
            "sample": f"layer-0 projections x{runs} ({layer_s * 1e3:.0f} ms/layer, recipe fp32 float path), head "
                      f"once ({head_s * 1e3:.0f} ms), attention over 4096 positions once ({attn_s * 1e3:.0f} ms, "
                      f"numpy), scaled to 32 layers; {cores} threads"}
    print(json.dumps(out), flush=True)
    graph.close()


def int8_bench(args):
    """recipe's int(8) sum (rqmv_matvec_int8) on a workload's weight, fp32
    activations: the same whole-job graph timing; kernel durations from events
    recorded around each launch; parity bit for bit against the oracle."""
    import rqmv
    from rqmv import synth

    fmt, rows, cols, _, desc = WORKLOADS[args.workload]
    m, step = args.m, args.int8
    desc = f"{desc}, recipe int(8) sum step {step}"
    log(f"bench: {args.workload} int8 step {step} M={m} steps={args.steps} warmup={args.warmup}")
    rqmv.init(0)
    w = synth.weights(fmt, rows, cols)
    x32 = synth.activations_f32(m * cols).reshape(m, cols)
    alg_bytes = w.nbytes + m * cols * 4 + m * rows * 4
    copies = args.copies or max(2, -(-2 * MALL_BYTES // w.nbytes) + 1)
    Ws = [rqmv.Weight(fmt, rows, cols, w) for _ in range(copies)]
    xb = rqmv.DeviceBuffer.from_array(x32)
    yb = rqmv.DeviceBuffer(4 * m * rows)
    stream = rqmv.Stream()
    exact = None
    if not args.no_check:
        import oracle

        rqmv.matvec_int8(Ws[0], xb, m, cols, yb, rows, step, stream=stream)
        stream.synchronize()
        y = yb.download(np.float32).reshape(m, rows)
        ref = oracle.int8_matvec(fmt, w, rows, cols, x32, step)
        exact = bool(np.array_equal(y.view(np.uint32), ref.view(np.uint32)))
        log(f"bench: int8 parity bit-exact {exact}")
        if not exact:
            sys.exit(1)

    def enqueue_steps(count):
        for i in range(count):
            rqmv.matvec_int8(Ws[i % copies], xb, m, cols, yb, rows, step, stream=stream)

    graph = rqmv.Graph(stream, lambda: enqueue_steps(args.steps))
    graph.launch(stream)
    stream.synchronize()
    e0, e1 = rqmv.Event(), rqmv.Event()
    e0.record(stream)
    graph.launch(stream)
    e1.record(stream)
    e1.synchronize()
    ms_per_step = e0.elapsed_ms(e1) / args.steps
    starts = [rqmv.Event() for _ in range(args.steps)]
    stops = [rqmv.Event() for _ in range(args.steps)]
    for i in range(args.steps):
        starts[i].record(stream)
        rqmv.matvec_int8(Ws[i % copies], xb, m, cols, yb, rows, step, stream=stream)
        stops[i].record(stream)
    stream.synchronize()
    ker_ms = float(np.mean([starts[i].elapsed_ms(stops[i]) for i in range(args.steps)]))
    log(f"bench: int8 graph {ms_per_step * 1e3:.2f} us/step, event-bracketed kernel {ker_ms * 1e3:.2f} us")
    achieved = alg_bytes / (ker_ms * 1e-3) / 1e9
    out = {
        "metric": "recipe int(8) sum matvec effective HBM GB/s at batch 1",
        "value": round(alg_bytes / (ms_per_step * 1e-3) / 1e9, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": desc, "format": fmt.upper(), "rows": rows, "cols": cols, "m": m, "step": step,
                   "activations": "f32", "weight_copies": copies, "bytes_per_step": alg_bytes,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "stream_copy": stream_copy(achieved),
        "kernel_us": round(ker_ms * 1e3, 3),
        "parity_bit_exact": exact,
    }
    if not args.no_cpu:
        import oracle

        from concurrent.futures import ThreadPoolExecutor

        cores, hostinfo = host_cpu()
        rb = w.nbytes // rows
        chunks = [(rows * c // cores, rows * (c + 1) // cores) for c in range(cores)]

        def part(r0, r1):
            return oracle.int8_matvec(fmt, w[r0 * rb:r1 * rb], r1 - r0, cols, x32, step)

        with ThreadPoolExecutor(cores) as pool:
            runs, t0 = 0, time.perf_counter()
            while True:
                list(pool.map(lambda c: part(*c), chunks))
                runs += 1
                el = time.perf_counter() - t0
                if el >= args.cpu_seconds:
                    break
        per = el / runs
        out["cpu_baseline"] = {"value": round(alg_bytes / per / 1e9, 3), "unit": "GB/s", "cores": cores,
                               "kind": "port", **hostinfo,
                               "sample": f"{runs} full int(8) matvecs in {el:.1f} s, {per * 1e3:.2f} ms each: the "
                                         f"oracle's restatement of the int(8) sum, rows split over {cores} threads"}
    print(json.dumps(out), flush=True)
    graph.close()


def grid_table(args):
    """The headline product beside a plain read of the same bytes, at the same
    grids, in one process: for each grid G in --grids, `args.steps` plain
    reads of 33 MB (a rotating window of a buffer >= 2x the Infinity Cache,
    256 threads per workgroup, --inflight loads in flight per thread;
    libmeasure.so) and `args.steps` Q4_K 4096->14336 products at one fp16
    activation row in the one-wave-per-tile form (RQMV_K2=0) with RQMV_GRID =
    G (rotating weight copies); then the product as planned (two waves per
    tile). Each dispatch is timed by events it records itself. Prints one
    JSON line with a row per (kernel, grid); profile the same command with
    rocprofv3 to read counters per dispatch."""
    import ctypes

    import rqmv
    from rqmv import synth

    fmt, rows, cols, _, desc = WORKLOADS["q4_k_up"]
    rqmv.init(0)
    w = synth.weights(fmt, rows, cols)
    nbytes = (w.nbytes + 15) // 16 * 16
    copies = args.copies or max(2, -(-2 * MALL_BYTES // nbytes) + 1)
    Ws = [rqmv.Weight(fmt, rows, cols, w) for _ in range(copies)]
    xb = rqmv.DeviceBuffer.from_array(synth.activations_f16(cols))
    yb = rqmv.DeviceBuffer(4 * rows)
    big = rqmv.DeviceBuffer(nbytes * copies)
    big.fill_zero()
    grids = [int(g) for g in args.grids.split(",")]
    sink = rqmv.DeviceBuffer(4 * 256 * max(grids))
    stream = rqmv.Stream()
    meas = ctypes.CDLL(os.path.join(ROOT, "recipe-dev_amd", "libmeasure.so"))
    meas.measure_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_void_p]
    alg = w.nbytes + 2 * cols + 4 * rows

    def timed(launch):
        for i in range(args.warmup):
            launch(i, None, None)
        stream.synchronize()
        ev = [(rqmv.Event(), rqmv.Event()) for _ in range(args.steps)]
        for i in range(args.steps):
            launch(i, ev[i][0].handle, ev[i][1].handle)
        stream.synchronize()
        d = np.array([a.elapsed_ms(b) for a, b in ev]) * 1e3
        for a, b in ev:
            a.close()
            b.close()
        return {"mean_us": round(float(d.mean()), 3), "median_us": round(float(np.median(d)), 3),
                "p10_us": round(float(np.percentile(d, 10)), 3), "p90_us": round(float(np.percentile(d, 90)), 3)}

    def mv(i, e0, e1):
        if e0 is None:
            Ws[i % copies].matvec(xb, rqmv.DTYPE_F16, 1, cols, yb, rows, stream)
        else:
            _check_mv(rqmv, Ws[i % copies], xb, yb, rows, cols, stream, e0, e1)

    table = []
    for g in grids:
        def read(i, e0, e1, g=g):
            rc = meas.measure_stream_read(big.ptr + (i % copies) * nbytes, nbytes, g, args.inflight, 0x9E3779B9,
                                          sink.ptr, stream.handle, e0, e1)
            if rc:
                raise RuntimeError(f"measure_stream_read: HIP error {rc}")

        r = timed(read)
        r.update({"kernel": "plain read", "grid": g, "bytes": nbytes,
                  "gbs": round(nbytes / (r["mean_us"] * 1e-6) / 1e9, 1)})
        log(f"bench: plain read grid {g}: {r}")
        table.append(r)
        os.environ["RQMV_GRID"] = str(g)
        os.environ["RQMV_K2"] = "0"
        r = timed(mv)
        r.update({"kernel": "matvec_int Q4_K 4096->14336 M=1 (one wave per tile)", "grid": g, "bytes": alg,
                  "gbs": round(alg / (r["mean_us"] * 1e-6) / 1e9, 1)})
        log(f"bench: matvec grid {g}: {r}")
        table.append(r)
        del os.environ["RQMV_GRID"]
        del os.environ["RQMV_K2"]
    r = timed(mv)
    r.update({"kernel": "matvec_int_k2 Q4_K 4096->14336 M=1 (as planned: two waves per tile)", "grid": 512,
              "threads": 512, "bytes": alg, "gbs": round(alg / (r["mean_us"] * 1e-6) / 1e9, 1)})
    log(f"bench: matvec as planned: {r}")
    table.append(r)
    print(json.dumps({"grid_table": table, "inflight": args.inflight, "copies": copies, "steps": args.steps}),
          flush=True)


def issue_rates(args):
    """Issue cost of single VALU opcodes on this GPU (libmeasure.so's probe):
    per opcode, `args.steps` launches of 2,048 workgroups x 256 threads, each
    lane running eight independent chains of 4,096 instructions, timed by
    events the dispatches record. Reports ns per wave-instruction per SIMD
    (the launch time over the wave-instructions each SIMD issues) and that in
    cycles at the clock the probe's plain 32-bit adds run at, taken as two
    cycles per wave64 instruction. Prints one JSON line."""
    import ctypes

    import rqmv

    rqmv.init(0)
    blocks, iters = 2048, 4096
    cus = 256  # MI355X (gfx950): 256 CUs of four SIMDs
    out = rqmv.DeviceBuffer(4 * 256 * blocks)
    stream = rqmv.Stream()
    meas = ctypes.CDLL(os.path.join(ROOT, "recipe-dev_amd", "libmeasure.so"))
    meas.measure_issue_name.restype = ctypes.c_char_p
    meas.measure_issue_rate.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p]
    wave_ops_per_simd = blocks * 4 * iters * 8 / (cus * 4)
    rows = []
    for op in range(meas.measure_issue_ops()):
        name = meas.measure_issue_name(op).decode()
        meas.measure_issue_rate(op, blocks, iters, out.ptr, stream.handle, None, None)
        ev = [(rqmv.Event(), rqmv.Event()) for _ in range(args.steps)]
        for a, b in ev:
            rc = meas.measure_issue_rate(op, blocks, iters, out.ptr, stream.handle, a.handle, b.handle)
            if rc:
                raise RuntimeError(f"measure_issue_rate: HIP error {rc}")
        stream.synchronize()
        us = float(np.median([a.elapsed_ms(b) for a, b in ev])) * 1e3
        for a, b in ev:
            a.close()
            b.close()
        rows.append({"opcode": name, "launch_us": round(us, 1),
                     "ns_per_wave_op": round(us * 1e3 / wave_ops_per_simd, 3)})
        log(f"bench: {rows[-1]}")
    base = next(r["ns_per_wave_op"] for r in rows if r["opcode"] == "v_add_u32")
    for r in rows:
        r["cycles_if_add_is_2"] = round(2.0 * r["ns_per_wave_op"] / base, 2)
    print(json.dumps({"issue_rates": rows, "blocks": blocks, "threads": 256, "chains": 8, "iters": iters,
                      "cus": cus, "launches": args.steps}), flush=True)


def _check_mv(rqmv, W, xb, yb, rows, cols, stream, e0, e1):
    rc = rqmv.lib().lib.rqmv_matvec_timed(W.handle, xb.ptr, rqmv.DTYPE_F16, 1, cols, yb.ptr, rows, stream.handle,
                                          e0, e1)
    if rc:
        raise RuntimeError(f"rqmv_matvec_timed: {rc}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="q4_k_up",
                    choices=sorted(WORKLOADS) + ["moe_c4", "decode_c5", "grid_table", "issue_rates"])
    ap.add_argument("--grids", default="512,1024,2048", help="grid_table: workgroup counts")
    ap.add_argument("--inflight", type=int, default=4, choices=[1, 2, 4, 8], help="grid_table: plain read loads in flight")
    ap.add_argument("--m", type=int, default=1, help="activation rows")
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0: enough to exceed 2x MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--int8", type=int, default=0, choices=[0, 32, 256],
                    help="run recipe's int(8) sum with this step instead (fp32 activations)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="only run a plain device copy of this many MB per step (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build runs the matvec on a "
              f"single MI355X; rows would shard across GPUs with no collective on the hot path)", file=sys.stderr)
        sys.exit(2)

    if args.copy_mb:
        copy_calibration(args.copy_mb, args.steps)
        return

    if args.workload == "moe_c4":
        moe_bench(args)
        return
    if args.workload == "decode_c5":
        decode_bench(args)
        return
    if args.workload == "issue_rates":
        issue_rates(args)
        return
    if args.workload == "grid_table":
        grid_table(args)
        return

    if args.int8:
        int8_bench(args)
        return

    import rqmv
    from rqmv import synth

    fmt, rows, cols, xdt, desc = WORKLOADS[args.workload]
    m = args.m
    log(f"bench: {args.workload} ({desc}) M={m} steps={args.steps} warmup={args.warmup}")
    rqmv.init(0)
    w = synth.weights(fmt, rows, cols)
    if xdt == "f16":
        xh = synth.activations_f16(m * cols).reshape(m, cols)
        x32 = synth.fp16_to_f32(xh)
        dtype_code, xbytes = rqmv.DTYPE_F16, 2
    else:
        xh = synth.activations_f32(m * cols).reshape(m, cols)
        x32 = xh
        dtype_code, xbytes = rqmv.DTYPE_F32, 4
    weight_bytes = w.nbytes
    alg_bytes = weight_bytes + m * cols * xbytes + m * rows * 4
    flops = 2.0 * m * rows * cols
    copies = args.copies or max(2, -(-2 * MALL_BYTES // weight_bytes) + 1)
    log(f"bench: {copies} weight copies of {weight_bytes / 1e6:.1f} MB")
    Ws = [rqmv.Weight(fmt, rows, cols, w) for _ in range(copies)]
    xb = rqmv.DeviceBuffer.from_array(xh)
    yb = rqmv.DeviceBuffer(4 * m * rows)
    stream = rqmv.Stream()

    rel = None
    if not args.no_check:
        import oracle

        Ws[0].matvec(xb, dtype_code, m, cols, yb, rows, stream)
        stream.synchronize()
        y = yb.download(np.float32).reshape(m, rows)
        ref = oracle.matvec_recipe_f32(fmt, w, rows, cols, x32, threads=8)
        rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
        log(f"bench: parity rel-L2 {rel:.3e}")
        if not rel <= 1e-3:
            log("bench: parity check failed")
            sys.exit(1)

    def enqueue_steps(count, start=0):
        for i in range(count):
            Ws[(start + i) % copies].matvec(xb, dtype_code, m, cols, yb, rows, stream)

    # whole job: K launches in one graph
    graph = rqmv.Graph(stream, lambda: enqueue_steps(args.steps))
    for _ in range(max(1, args.warmup // max(1, args.steps) + 1)):
        graph.launch(stream)
    stream.synchronize()
    e0, e1 = rqmv.Event(), rqmv.Event()
    e0.record(stream)
    graph.launch(stream)
    e1.record(stream)
    e1.synchronize()
    total_ms = e0.elapsed_ms(e1)
    ms_per_step = total_ms / args.steps
    log(f"bench: graph {args.steps} steps {total_ms:.3f} ms -> {ms_per_step * 1e3:.2f} us/step")

    # kernel durations: each dispatch records its own start/stop events
    enqueue_steps(args.warmup)
    stream.synchronize()
    starts = [rqmv.Event() for _ in range(args.steps)]
    stops = [rqmv.Event() for _ in range(args.steps)]
    for i in range(args.steps):
        Ws[i % copies].matvec_timed(xb, dtype_code, m, cols, yb, rows, stream, starts[i], stops[i])
    stream.synchronize()
    ker = np.array([starts[i].elapsed_ms(stops[i]) for i in range(args.steps)])
    ker_ms = float(ker.mean())
    log(f"bench: kernel mean {ker_ms * 1e3:.2f} us, median {np.median(ker) * 1e3:.2f} us, "
        f"p10 {np.percentile(ker, 10) * 1e3:.2f} p90 {np.percentile(ker, 90) * 1e3:.2f}")

    achieved = alg_bytes / (ker_ms * 1e-3) / 1e9
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if xdt == "f16" else "f32",
        "data": "synthetic",
        "config": {"workload": desc, "format": fmt.upper(), "rows": rows, "cols": cols, "m": m,
                   "activations": xdt, "accumulate": "f32", "weight_copies": copies,
                   "bytes_per_step": alg_bytes, "flops_per_step": flops, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(args.workload, m),
                     "timing": "mean of per-dispatch start/stop events recorded by each launch itself "
                               "(hipExtLaunchKernelGGL), live in this run",
                     "rocprof": rocprof_roofline(args.workload, m, alg_bytes)},
        "stream_copy": stream_copy(achieved),
        "kernel_us": round(ker_ms * 1e3, 3),
        "kernel_us_median": round(float(np.median(ker)) * 1e3, 3),
        "kernel_us_p10": round(float(np.percentile(ker, 10)) * 1e3, 3),
        "kernel_us_p90": round(float(np.percentile(ker, 90)) * 1e3, 3),
        "gflops": round(flops / (ker_ms * 1e-3) / 1e9, 1),
        "parity_rel_l2": rel,
    }
    mfma = _profile_entry("mfma_util.json", f"{args.workload}_m{m}")
    if mfma:
        out["mfma"] = {"util": mfma["mfma_util"], "tflops_under_counters": mfma["tflops"],
                       "kernel_us_under_counters": mfma["kernel_us_under_counters"],
                       "source": mfma.get("source", "profiles/mfma_util.json"),
                       "definition": "SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs)"}
    if not args.no_cpu:
        log("bench: cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(fmt, rows, cols, x32, args.cpu_seconds, w, alg_bytes)
    print(json.dumps(out), flush=True)
    graph.close()


if __name__ == "__main__":
    main()
