#!/usr/bin/env python3
"""Batch-1 decode through a full DeepSeek-R1-shape MoE layer on one MI355X.

One step = one token through the MoE branch of a layer (router logits ->
route -> 8 routed experts + 1 shared expert -> combine -> residual), via
the library's C ABI (fdm_moe_layer).  Every step uses a different seeded
token and the next of `--layers` resident layers (round robin), so the
256 MB Infinity Cache cannot serve the weights: each step streams its
experts from HBM.  All inputs are already resident when timing starts.

Prints one JSON line (rank 0):
  value        microseconds per token (lower is better)
  layer_gbps   algorithmic bytes per token / time per token
  roofline     the layer kernel (router, route, 9 experts, combine in one
               launch), timed live with HIP events on the launch stream
  cpu_baseline the reference's CPU expert path (C restatement) on this
               host's cores, on a bounded sample of the same workload
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "Q4_K MoE layer µs/token (batch 1) + achieved HBM GB/s as % of ~8 TB/s peak"
HBM_PEAK_GBPS = 8000.0

# Algorithmic bytes (weights actually required + fp32 activations in/out).
GATE_BYTES = 57344 * 144                     # one Q4_K 2048 x 7168 matrix
DOWN_BYTES = {"q4k": 57344 * 144, "q6k": 57344 * 210}
ROUTER_BYTES = 256 * 7168 * 4 + 256 * 4      # W_g + bias
HIDDEN, FFN = 7168, 2048
FDM_STREAM_LAYER = 60  # the streamed layer of the stream leg (the resident ones are 3 ..)
COPY_BYTES = 256 << 20   # calibration copy of the counter passes


def layer_bytes(down, K=8):
    slots = K + 1
    weights = slots * (2 * GATE_BYTES + DOWN_BYTES[down]) + ROUTER_BYTES
    acts = HIDDEN * 4 * 3  # h_post, h_in in; hidden out
    return weights + acts


def percentiles(us):
    """median, p10, p90 of a list of microsecond timings."""
    a = sorted(us)
    pick = lambda q: a[min(len(a) - 1, int(round(q * (len(a) - 1))))]
    return {"median_us": round(pick(0.5), 3), "p10_us": round(pick(0.1), 3), "p90_us": round(pick(0.9), 3)}


def event_times(torch, fn, n):
    """fn(i) for i < n, each bracketed by HIP events on torch's current stream
    (the stream the library launches on); per-call microseconds."""
    st = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        st[i].record()
        fn(i)
        en[i].record()
    torch.cuda.synchronize()
    return [st[i].elapsed_time(en[i]) * 1e3 for i in range(n)]


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_profile_json(name, key):
    """A summary committed under profiles/ (rocprofv3 counters), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def load_traffic(kernel, workload):
    """HBM bytes per launch measured by rocprofv3 counters (profiles/)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel, {}).get(workload)
    except (OSError, ValueError):
        return None


def cpu_baseline(down, seconds, K=8):
    """Median us/token of the two CPU versions of the layer on bounded
    samples of the same workload: the reference-shaped path (one thread per
    expert, full fp32 dequant then sgemv) and the tuned one (fused row
    dequant-dot over every host core)."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    q6 = down == "q6k"
    blobs = [O.synth_expert(900 + i, down_is_q6=q6) for i in range(K + 1)]
    Wg = O.synth_normal(256 * HIDDEN, 0.0, 0.01, 901).reshape(256, HIDDEN)
    bias = O.synth_normal(256, 0.0, 0.1, 902)
    x = O.synth_normal(HIDDEN, 0.0, 1.0, 903)
    h_in = O.synth_normal(HIDDEN, 0.0, 1.0, 904)
    model = cpu_model()
    t0 = time.perf_counter()
    O.cpu_layer_baseline(blobs, q6, Wg, bias, x, h_in, 2)
    per = max(time.perf_counter() - t0, 1e-3) / 2
    reps = int(max(3, min(200, seconds / per)))
    us, _ = O.cpu_layer_baseline(blobs, q6, Wg, bias, x, h_in, reps)
    ref = {
        "value": round(us, 1),
        "unit": "us/token",
        "cores": K + 1,
        "kind": "port",
        "sample": (f"{reps} tokens through one R1 MoE layer on the host ({model}, {os.cpu_count()} CPUs "
                   f"visible): router sgemv + route() + {K} routed and 1 shared expert, each "
                   f"dequantised to fp32 and run as 3 sgemv + SiLU*mul on its own thread "
                   f"(infer.m:1878-1922, USE_CPU_EXPERTS), {down.upper()} down; median per token"),
    }
    t0 = time.perf_counter()
    O.cpu_layer_tuned(blobs, q6, Wg, bias, x, h_in, 2)
    per = max(time.perf_counter() - t0, 1e-3) / 2
    reps = int(max(3, min(2000, seconds / per)))
    us, _, threads = O.cpu_layer_tuned(blobs, q6, Wg, bias, x, h_in, reps)
    tuned = {
        "value": round(us, 1),
        "unit": "us/token",
        "cores": threads,
        "kind": "port",
        "sample": (f"{reps} tokens through the same layer on {threads} host threads ({model}): rows "
                   f"dequantised and dotted in one pass (AVX2 FMA), no fp32 matrix copies; "
                   f"median per token"),
    }
    return ref, tuned


def bench_read_ceiling(F, torch, args, stream, K, h_post, h_in):
    """Per step: fdm_layer_read_ceiling over the step's rotated layer with K
    distinct seeded expert ids; wall time per step (back-to-back launches, as
    the headline) and the per-launch HIP-event average."""
    rng = np.random.default_rng(4321)
    n = args.warmup + args.steps
    ids = np.stack([rng.choice(256, K, replace=False) for _ in range(n)]).astype(np.int32)
    d_ids = torch.from_numpy(ids).cuda()
    sink = torch.empty(HIDDEN, dtype=torch.int32, device="cuda")
    run = lambda i: F.layer_read_ceiling(3 + i % args.layers, d_ids[i], K, h_post[i], h_in[i], sink,
                                         stream=stream)
    for i in range(args.warmup):
        run(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup, n):
        run(i)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / args.steps * 1e6
    F.prof_enable(True)
    F.prof_reset()
    for i in range(args.warmup, n):
        run(i)
    torch.cuda.synchronize()
    cnt, tot, mn, mx = F.prof_read("ceiling")
    F.prof_enable(False)
    return {"us_per_step": round(us, 2), "kernel_avg_us": round(tot / max(cnt, 1) * 1e3, 2)}


def bench_matvec(F, torch, args, n_sets=64, calls=256):
    """Config 0: y = W x for a Q4_K W [2048 x 7168] (the dequant_matvec_q4k
    of one gate matrix) over n_sets distinct weight sets (> the 256 MB
    Infinity Cache), a new set each call; per-call HIP events."""
    from flash_deepseek_amd.synthetic import make_tokens
    rows, cols = 2048, 7168
    nb = rows * cols // 256
    W = torch.empty(n_sets * nb * 144, dtype=torch.uint8, device="cuda")
    for i in range(n_sets):
        F.synth_q4k(W.data_ptr() + i * nb * 144, nb, 5000 + i)
    x = make_tokens(1, 5100)[0]
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    run = lambda i: F.matvec_q4k(W.data_ptr() + (i % n_sets) * nb * 144, x, y, rows, cols)
    for i in range(16):
        run(i)
    us = event_times(torch, run, calls)
    del W
    nbytes = nb * 144 + cols * 4 + rows * 4
    r = {"workload": "Q4_K matvec 2048x7168, batch 1 (fdm_matvec_q4k: one launch, x staged per workgroup, "
                     "fp32 group dots)",
         "weight_sets": n_sets, "calls": calls, "bytes_per_call": nbytes}
    r.update(percentiles(us))
    r["gbps"] = round(nbytes / (r["median_us"] * 1e-6) / 1e9, 1)
    r["frac"] = round(r["gbps"] / HBM_PEAK_GBPS, 4)
    return r


def bench_expert(F, torch, down, n_sets=64, calls=256):
    """Config 1: one SwiGLU expert at batch 1 (fdm_expert_ffn on the packed
    blob) over n_sets distinct experts, a new one each call."""
    from flash_deepseek_amd.synthetic import fill_blob, make_tokens
    q6 = down == "q6k"
    es = F.EXPERT_Q6K_BYTES if q6 else F.EXPERT_Q4K_BYTES
    blobs = torch.empty(n_sets * es, dtype=torch.uint8, device="cuda")
    for i in range(n_sets):
        fill_blob(blobs, i * es, 6000 + i, 0, q6)
    x = make_tokens(1, 6100)[0]
    out = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    run = lambda i: F.expert_ffn(blobs.data_ptr() + (i % n_sets) * es, es, x, out)
    for i in range(16):
        run(i)
    us = event_times(torch, run, calls)
    del blobs
    nbytes = es + HIDDEN * 4 * 2 + FFN * 4 * 2
    r = {"workload": f"one SwiGLU expert, batch 1: Q4_K gate/up 2048x7168, {down.upper()} down 7168x2048 "
                     "(fdm_expert_ffn)", "weight_sets": n_sets, "calls": calls, "bytes_per_call": nbytes}
    r.update(percentiles(us))
    r["gbps"] = round(nbytes / (r["median_us"] * 1e-6) / 1e9, 1)
    r["frac"] = round(r["gbps"] / HBM_PEAK_GBPS, 4)
    return r


def bench_layer_q6k(F, torch, args, stream, K, n_layers=6, steps=200):
    """The batch-1 layer with Q6_K down matrices (k_layer_q6k), n_layers
    resident layers rotated, a new token per step; per-step HIP events."""
    from flash_deepseek_amd.synthetic import make_layer, make_tokens
    keep = []
    for l in range(n_layers):
        lay = make_layer(700 + l, down_q6=True)
        F.attach_layer(40 + l, lay.experts, lay.expert_size, lay.Wg, lay.bias, lay.shared)
        lay.experts = lay.shared = None
        keep.append(lay)
    torch.cuda.empty_cache()
    h = make_tokens(steps + 20, 7101)
    h_in = make_tokens(steps + 20, 7102)
    out = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    run = lambda i: F.moe_layer(40 + i % n_layers, h[i], h_in[i], K, out, stream=stream)
    for i in range(20):
        run(i)
    us = event_times(torch, lambda i: run(20 + i), steps)
    F.sync(stream)
    for l in range(n_layers):
        F.release_layer(40 + l)
    nbytes = layer_bytes("q6k", K)
    r = {"workload": "the batch-1 layer with Q6_K down (k_layer_q6k)", "layers_rotated": n_layers,
         "steps": steps, "bytes_per_token": nbytes}
    r.update(percentiles(us))
    r["gbps"] = round(nbytes / (r["median_us"] * 1e-6) / 1e9, 1)
    r["frac"] = round(r["gbps"] / HBM_PEAK_GBPS, 4)
    return r


def bench_norm(F, torch, args, stream, K, steps=200):
    """rms_norm on the device (fdm_rms_norm: one token of 7168, and 512
    tokens), and the batch-1 layer with the rms_norm fused into its launch
    (fdm_moe_layer_norm) over the same rotated layers as the headline, each
    timed per call with HIP events."""
    from flash_deepseek_amd.synthetic import make_tokens
    out = {}
    w = make_tokens(1, 7301)[0]
    for T in (1, 512):
        x = make_tokens(T, 7302 + T)
        o = torch.empty_like(x)
        for _ in range(10):
            F.rms_norm(x, w, o, T, stream=stream)
        us = event_times(torch, lambda i: F.rms_norm(x, w, o, T, stream=stream), steps)
        r = percentiles(us)
        r["bytes"] = 2 * T * HIDDEN * 4 + HIDDEN * 4
        out[f"rms_norm_t{T}"] = r
    h = make_tokens(steps + 20, 7303)
    hid = torch.empty((steps + 20, HIDDEN), dtype=torch.float32, device="cuda")
    run = lambda i: F.moe_layer_norm(3 + i % args.layers, h[i], w, K, hid[i], stream=stream)
    for i in range(20):
        run(i)
    us = event_times(torch, lambda i: run(20 + i), steps)
    F.sync(stream)
    r = {"workload": "the batch-1 layer with its rms_norm fused in (hidden state in, rms_norm + "
                     "router + route + 8 routed and 1 shared expert + combine + residual)",
         "layers_rotated": args.layers, "steps": steps}
    r.update(percentiles(us))
    out["layer_with_rms_norm"] = r
    return out


def bench_batched(F, torch, layers, args, stream, K, steps=20, warmup=3):
    """Batched decode through the resident layers: per token count T, the
    mean over `steps` steps (new seeded tokens each, next layer each)."""
    from flash_deepseek_amd.synthetic import make_tokens
    out = {}
    es = layers[0].expert_size
    for T in [int(t) for t in args.batched.split(",") if t]:
        X = make_tokens((steps + warmup) * T, 8100 + T).reshape(steps + warmup, T, HIDDEN)
        Hin = make_tokens((steps + warmup) * T, 8200 + T).reshape(steps + warmup, T, HIDDEN)
        Y = torch.empty((T, HIDDEN), dtype=torch.float32, device="cuda")
        nd = torch.zeros(steps + warmup, dtype=torch.int32, device="cuda")
        for i in range(steps + warmup):
            if i == warmup:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
            F.moe_forward_batched(3 + i % args.layers, X[i], Hin[i], T, K, Y,
                                  n_distinct=nd[i:i + 1], stream=stream)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        d_mean = float(nd[warmup:].float().mean().item())
        step_bytes = (d_mean + 1) * es + ROUTER_BYTES + T * HIDDEN * 4 * 3
        out[str(T)] = {"us_per_token": round(dt / T * 1e6, 2), "ms_per_step": round(dt * 1e3, 4),
                       "distinct_experts": round(d_mean, 1),
                       "gbps": round(step_bytes / dt / 1e9, 1),
                       "frac": round(step_bytes / dt / 1e9 / HBM_PEAK_GBPS, 4)}
    return out


def bench_prefill(F, torch, layers, args, stream, K, n_layers=4, iters=5):
    """Prefill of args.prefill tokens through n_layers resident layers
    (h <- h + MoE(rms_norm(h, w)) per layer, in place); each timed iteration
    starts from the same seeded activations."""
    from flash_deepseek_amd.synthetic import make_tokens
    T = args.prefill
    H0 = make_tokens(T, 9100)
    H = torch.empty_like(H0)
    norms = [make_tokens(1, 9200 + l, mean=1.0, std=0.1)[0] for l in range(n_layers)]
    ids = [3 + l for l in range(n_layers)]
    nd = []
    times = []
    for i in range(iters + 1):
        H.copy_(H0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        F.moe_prefill(ids, H, T, K, norms, stream=stream)
        torch.cuda.synchronize()
        if i:
            times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    es = layers[0].expert_size
    # every layer reads its selected experts (nearly all 256 at this T) + shared + router
    idx = torch.empty((n_layers, T, K), dtype=torch.int32, device="cuda")
    H.copy_(H0)
    F.moe_prefill(ids, H, T, K, norms, idx=idx, stream=stream)
    torch.cuda.synchronize()
    d = [len(torch.unique(idx[l])) for l in range(n_layers)]
    step_bytes = sum((dl + 1) * es for dl in d) + n_layers * (ROUTER_BYTES + T * HIDDEN * 4 * 2)
    flops = n_layers * T * (K + 1) * 3 * 2 * HIDDEN * FFN
    out = {"tokens": T, "layers": n_layers, "ms": round(dt * 1e3, 3),
           "tokens_per_s": round(T / dt, 1), "distinct_experts": d,
           "gbps": round(step_bytes / dt / 1e9, 1),
           "frac": round(step_bytes / dt / 1e9 / HBM_PEAK_GBPS, 4),
           "tflops": round(flops / dt / 1e12, 2),
           "mfma_flops_frac": round(flops / dt / 2.5e15, 4),
           "note": ("the stack chains the synthetic layers as the workload states; their Q4_K weights "
                    "have a positive mean, so the residual grows by orders of magnitude per layer and "
                    "layers 2-4 route the tokens onto few experts (distinct_experts); "
                    "per_layer_fresh below times each layer on fresh N(0,1) tokens")}
    # each layer alone on fresh tokens: the routing spread of a real prompt
    fresh = [make_tokens(T, 9300 + l) for l in range(n_layers)]
    ft, fd = [], []
    for rep in range(3):
        for l in range(n_layers):
            H.copy_(fresh[l])
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            F.moe_prefill([ids[l]], H, T, K, [norms[l]], idx=idx[l], stream=stream)
            torch.cuda.synchronize()
            if rep:
                ft.append(time.perf_counter() - t0)
            if rep == 2:
                fd.append(len(torch.unique(idx[l])))
    lt = sorted(ft)[len(ft) // 2]
    fbytes = sum(dl + 1 for dl in fd) / n_layers * es + ROUTER_BYTES + T * HIDDEN * 4 * 2
    out["per_layer_fresh"] = {"ms_per_layer": round(lt * 1e3, 3), "distinct_experts": fd,
                              "tokens_per_s_4_layers": round(T / (lt * n_layers), 1),
                              "gbps": round(fbytes / lt / 1e9, 1),
                              "frac": round(fbytes / lt / 1e9 / HBM_PEAK_GBPS, 4)}
    mf = load_profile_json("mfma.json", "prefill_512tok")
    if mf:
        out["mfma_counters"] = mf
    return out


def bench_dense(F, torch, args, stream, steps=60, warmup=6):
    """Dense FFN layers 0..n-1 (R1: 3 layers, F16 weights, inter 18432):
    hidden = h_in + W_down (silu(W_gate h) * (W_up h)) per call, the next
    layer each call (each layer's 792 MB exceeds the 256 MB MALL)."""
    from flash_deepseek_amd.synthetic import make_tokens
    inter = F.DENSE_FFN
    g = torch.Generator(device="cuda").manual_seed(4242)
    for l in range(args.dense):
        mats = [(torch.randn((inter, HIDDEN), generator=g, device="cuda") * HIDDEN ** -0.5).half(),
                (torch.randn((inter, HIDDEN), generator=g, device="cuda") * HIDDEN ** -0.5).half(),
                (torch.randn((HIDDEN, inter), generator=g, device="cuda") * inter ** -0.5).half()]
        F.attach_dense(l, *mats, inter)  # the library keeps its own copy
        del mats
    torch.cuda.empty_cache()
    X = make_tokens(steps + warmup, 9300)
    Hin = make_tokens(steps + warmup, 9400)
    Y = torch.empty((steps + warmup, HIDDEN), dtype=torch.float32, device="cuda")
    for i in range(warmup):
        F.dense_ffn(i % args.dense, X[i], Hin[i], Y[i], stream=stream)
    torch.cuda.synchronize()
    F.prof_enable(True)
    F.prof_reset()
    t0 = time.perf_counter()
    for i in range(warmup, steps + warmup):
        F.dense_ffn(i % args.dense, X[i], Hin[i], Y[i], stream=stream)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    n, tot, mn, mx = F.prof_read("dense")
    F.prof_enable(False)
    for l in range(args.dense):
        F.release_dense(l)
    layer_bytes = 3 * inter * HIDDEN * 2 + HIDDEN * 4 * 3
    kern = tot / n * 1e-3 if n else dt
    return {"layers": args.dense, "inter": inter, "us_per_layer": round(dt * 1e6, 2),
            "kernel_avg_us": round(kern * 1e6, 2), "bytes_per_layer": layer_bytes,
            "gbps": round(layer_bytes / kern / 1e9, 1),
            "frac": round(layer_bytes / kern / 1e9 / HBM_PEAK_GBPS, 4)}


def bench_stream(F, torch, args, stream, K, tokens=24):
    """Streamed layer (fdm_moe_layer_streamed): the 256 routed experts stay in
    a layer file in the packed layout, held in the host page cache (written
    here, so every read is a page-cache hit), and are read into an HBM cache
    of n_cache slots on demand.  Per call: route on the device, the ids to the
    host, the shared expert and the cache hits launched at once, each miss's
    kernels queued behind its own chunk copies as its last chunk is read
    (32 reader threads), combine.  Host wall clock per synchronized call.
    n_cache 8: a new seeded token per call (nearly every expert a miss);
    n_cache 256: the warm-up tokens again (every expert a hit)."""
    import shutil
    import tempfile
    from flash_deepseek_amd.synthetic import make_layer, make_tokens
    lay = make_layer(901, down_q6=(args.down == "q6k"))
    es = lay.expert_size
    need = 256 * es
    folder = None
    for cand in ("/dev/shm", tempfile.gettempdir()):
        try:
            if shutil.disk_usage(cand).free > need + (1 << 30):
                folder = cand
                break
        except OSError:
            pass
    if folder is None:
        return {"skipped": f"no folder with {need / 1e9:.1f} GB free for the layer file"}
    fd, path = tempfile.mkstemp(prefix="fdm_layer_", suffix=".bin", dir=folder)
    out = {"layer_file_bytes": need, "expert_bytes": es, "K": K, "reader_threads": 32, "folder": folder}
    try:
        with os.fdopen(fd, "wb") as f:
            for e0 in range(0, 256, 16):
                f.write(lay.experts[e0 * es:(e0 + 16) * es].cpu().numpy().tobytes())
        lay.experts = None
        torch.cuda.empty_cache()
        L = FDM_STREAM_LAYER
        hid = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
        warm = 4
        for n_cache in (8, 256):
            F.stream_layer(L, path, es, lay.Wg, lay.bias, lay.shared, n_cache=n_cache, n_threads=32)
            try:
                hp = make_tokens(warm + tokens, 9100 + n_cache)
                hi = make_tokens(warm + tokens, 9200 + n_cache)
                for i in range(warm):
                    F.moe_layer_streamed(L, hp[i], hi[i], K, hid, stream=stream)
                torch.cuda.synchronize()
                pick = (lambda i: i % warm) if n_cache == 256 else (lambda i: warm + i)
                h0, m0, b0 = F.stream_stats(L)
                ms = []
                for i in range(tokens):
                    t0 = time.perf_counter()
                    F.moe_layer_streamed(L, hp[pick(i)], hi[pick(i)], K, hid, stream=stream)
                    torch.cuda.synchronize()
                    ms.append((time.perf_counter() - t0) * 1e3)
                F.sync(stream)
                h1, m1, b1 = F.stream_stats(L)
                r = {"tokens": tokens, "misses_per_token": round((m1 - m0) / tokens, 2),
                     "hits_per_token": round((h1 - h0) / tokens, 2),
                     "expert_mb_read_per_token": round((b1 - b0) / tokens / 1e6, 1)}
                a = sorted(ms)
                r["ms_per_token"] = {"median": round(a[len(a) // 2], 3), "p10": round(a[len(a) // 10], 3),
                                     "p90": round(a[(9 * len(a)) // 10], 3)}
                tot_s = sum(ms) / 1e3
                r["expert_read_gbps"] = round((b1 - b0) / tot_s / 1e9, 2) if tot_s > 0 else 0.0
                out[f"n_cache_{n_cache}"] = r
            finally:
                F.release_layer(L)
    finally:
        os.unlink(path)
    return out


def bench_attn(F, torch, args, stream, steps=50, K=8):
    """MLA attention of decode tokens (one layer, R1 shapes, F16 weights) at
    a cache of args.attn positions: the cache is filled first, then `steps`
    tokens are timed (positions args.attn .. args.attn + steps - 1).  Then
    the reference's whole MoE decode layer (layer_forward, infer.m:1837-1924)
    as one chain per token, for `steps` more tokens: attention with its
    residual (fdm_attn_forward), then rms_norm + router + route + experts +
    combine + residual in one launch (fdm_moe_layer_norm, over the rotated
    resident MoE layers), in place on the token's hidden state."""
    g = torch.Generator(device="cuda").manual_seed(766)

    def f16(rows, cols, *lead):
        t = torch.randn((*lead, rows, cols), generator=g, device="cuda") * cols ** -0.5
        return t.half().cpu().numpy().view(np.uint16)

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device="cuda")).cpu().numpy()

    w = {"attn_norm": norm(HIDDEN), "q_a": f16(1536, HIDDEN), "q_a_norm": norm(1536),
         "q_b": f16(128 * 192, 1536), "kv_a": f16(576, HIDDEN), "kv_a_norm": norm(512),
         "k_b": f16(512, 128, 128), "v_b": f16(128, 512, 128), "o_proj": f16(HIDDEN, 128 * 128)}
    S = args.attn
    F.attn_upload(0, w, max_seq=S + 2 * steps)
    wbytes = sum(a.nbytes for a in w.values())
    X = torch.randn((S + 2 * steps, HIDDEN), generator=g, device="cuda")
    for pos in range(S):
        F.attn_forward(0, X[pos], pos, stream=stream)
    torch.cuda.synchronize()
    F.prof_enable(True)
    F.prof_reset()
    t0 = time.perf_counter()
    for pos in range(S, S + steps):
        F.attn_forward(0, X[pos], pos, stream=stream)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    n, tot, mn, mx = F.prof_read("attn")
    F.prof_enable(False)
    kern = tot / n * 1e-3 if n else dt
    step_bytes = wbytes + (S + steps // 2) * 576 * 4 * 3
    out = {"cache_len": S, "us_per_token": round(dt * 1e6, 2), "kernels_us": round(kern * 1e6, 2),
           "weight_bytes": wbytes, "gbps": round(step_bytes / kern / 1e9, 1),
           "frac": round(step_bytes / kern / 1e9 / HBM_PEAK_GBPS, 4)}
    # the whole decode layer, chained per token on one stream
    nw = (1.0 + 0.1 * torch.randn(HIDDEN, generator=g, device="cuda")).contiguous()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i, pos in enumerate(range(S + steps, S + 2 * steps)):
        F.attn_forward(0, X[pos], pos, stream=stream)
        F.moe_layer_norm(3 + i % args.layers, X[pos], nw, K, X[pos], stream=stream)
    torch.cuda.synchronize()
    F.sync(stream)
    dl = (time.perf_counter() - t0) / steps
    F.attn_release(0)
    out["decode_layer"] = {
        "workload": "layer_forward of a MoE layer at batch 1: MLA attention at this cache length + residual, "
                    "then rms_norm + router + route + 8 routed and 1 shared expert + combine + residual "
                    f"({args.layers} resident MoE layers rotated), in place, chained on one stream",
        "tokens": steps, "us_per_token": round(dl * 1e6, 2)}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--layers", type=int, default=12, help="resident layers rotated per step")
    ap.add_argument("--down", choices=["q4k", "q6k"], default="q4k")
    ap.add_argument("--prof-steps", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded sample of each CPU baseline (seconds of host work)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--batched", default="16,64,256",
                    help="also time batched decode at these token counts ('' to skip)")
    ap.add_argument("--prefill", type=int, default=512,
                    help="also time prefill of this many tokens through 4 resident layers (0 to skip)")
    ap.add_argument("--attn", type=int, default=1024,
                    help="also time MLA attention of decode tokens at this KV cache length (0 to skip)")
    ap.add_argument("--dense", type=int, default=3,
                    help="also time the dense FFN over this many F16 dense layers (0 to skip)")
    ap.add_argument("--stream", type=int, default=1,
                    help="also time a streamed layer from a page-cached layer file, K = 8, with 8 "
                         "and 256 cache slots (0 to skip)")
    ap.add_argument("--configs", type=int, default=1,
                    help="also time the single matvec, the single expert (Q4_K and Q6_K down) "
                         "and the Q6_K-down layer (0 to skip)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="counter-collection run: a few layer steps, 8 batched-decode steps "
                         "of 256 tokens, then plain 256 MiB copies (read + write of known size) "
                         "that calibrate the counters")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on exactly one GPU (asked for {max(args.gpus, world)}): this "
              "build measures the hot path on one MI355X; multi-GPU sharding is a design "
              "note, not a measured configuration.", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, ROOT)
    import flash_deepseek_amd as F
    from flash_deepseek_amd.synthetic import make_layer, make_tokens

    K = 8
    F.init(0)
    stream = torch.cuda.current_stream().cuda_stream
    layers = []
    for l in range(args.layers):
        lay = make_layer(1 + l, down_q6=(args.down == "q6k"))
        F.attach_layer(3 + l, lay.experts, lay.expert_size, lay.Wg, lay.bias, lay.shared)
        # the library keeps its own resident copy of the experts; the router
        # weights and bias stay borrowed from `lay`
        lay.experts = lay.shared = None
        layers.append(lay)
    torch.cuda.empty_cache()
    n_tok = args.warmup + max(args.steps, args.prof_steps)
    h_post = make_tokens(n_tok, 7001)
    h_in = make_tokens(n_tok, 7002)
    out = torch.empty((n_tok, HIDDEN), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        F.moe_layer(3 + i % args.layers, h_post[i], h_in[i], K, out[i], stream=stream)

    if args.pmc_workload:
        for i in range(min(n_tok, 40)):
            step(i)
        # batched decode at 256 tokens (the grouped GEMMs' traffic), 8 steps
        # over the rotated layers, with each step's distinct-expert count
        bT, bsteps = 256, 8
        bX = make_tokens(bsteps * bT, 8356).reshape(bsteps, bT, HIDDEN)
        bH = make_tokens(bsteps * bT, 8357).reshape(bsteps, bT, HIDDEN)
        bY = torch.empty((bT, HIDDEN), dtype=torch.float32, device="cuda")
        bnd = torch.zeros(bsteps, dtype=torch.int32, device="cuda")
        for i in range(bsteps):
            F.moe_forward_batched(3 + i % args.layers, bX[i], bH[i], bT, K, bY, n_distinct=bnd[i:i + 1],
                                  stream=stream)
        n = COPY_BYTES // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # one elementwise kernel: reads and writes 256 MiB
        torch.cuda.synchronize()
        print(json.dumps({"pmc_workload": True, "layer_steps": min(n_tok, 40),
                          "batched_T": bT, "batched_distinct_experts": bnd.tolist(),
                          "expert_size": layers[0].expert_size,
                          "copy_bytes": COPY_BYTES, "copies": 3}), flush=True)
        return

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.steps):
        step(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    F.sync(stream)  # raises if a wait inside a layer kernel gave up
    us_per_token = elapsed / args.steps * 1e6

    # per-kernel durations from HIP events on the launch stream
    F.prof_enable(True)
    F.prof_reset()
    for i in range(args.warmup, args.warmup + args.prof_steps):
        step(i)
    torch.cuda.synchronize()
    F.sync(stream)
    phases = {}
    for name in ("layer",):
        n, tot, mn, mx = F.prof_read(name)
        phases[name] = {"launches": n, "avg_us": round(tot / max(n, 1) * 1e3, 2),
                        "min_us": round(mn * 1e3, 2), "max_us": round(mx * 1e3, 2)}
    F.prof_enable(False)
    # per-step HIP events over the same steps: the spread of the step time
    step_us = event_times(torch, lambda i: step(args.warmup + i), args.prof_steps)
    F.sync(stream)

    # the streaming ceiling of the same bytes: one dependency-free launch per
    # step that reads what the step's layer launch reads (router, 8 routed
    # experts -- distinct seeded ids per step --, the shared expert, h_post,
    # h_in) with the layer kernel's load policy, nothing else
    ceiling = bench_read_ceiling(F, torch, args, stream, K, h_post, h_in)

    lb = layer_bytes(args.down, K)
    k_us = phases["layer"]["avg_us"]
    achieved = lb / (k_us * 1e-6) / 1e9 if k_us > 0 else 0.0
    layer_gbps = lb / (us_per_token * 1e-6) / 1e9
    result = {
        "metric": METRIC,
        "value": round(us_per_token, 2),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_token / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4k weights x fp32 activations as three int8 digits (fp32 grade), dot4 -> fp32",
        "data": "synthetic (seeded, device-generated; no real weights)",
        "config": {
            "workload": ("DeepSeek-R1 MoE layer, batch-1 decode: fp32 router 256x7168 + "
                         "group-limited top-8 + 8 routed and 1 shared SwiGLU expert "
                         f"(Q4_K gate/up 2048x7168, {args.down.upper()} down 7168x2048), "
                         "combine + residual; 256 experts resident per layer; "
                         f"{args.layers} layers rotated per step "
                         f"({round(args.layers * (256 + 1) * layers[0].expert_size / 1e9, 1)} GB "
                         "resident), a new seeded token per step"),
        },
        "step_us": percentiles(step_us),
        "layer_bytes": lb,
        "layer_gbps": round(layer_gbps, 1),
        "layer_frac": round(layer_gbps / HBM_PEAK_GBPS, 4),
        "phases_us": phases,
        "roofline": {
            "kernel": "k_layer (router + route + 8 routed and 1 shared expert + combine)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": load_traffic("k_layer", f"deepseek_r1_batch1_{args.down}"),
            "traffic_source": ("HBM bytes per launch from the rocprofv3 FETCH_SIZE + WRITE_SIZE passes "
                               "committed in profiles/ (traffic.json), not measured in this run"),
            "bytes_per_launch": lb,
            "stream_ceiling": {
                "kernel": "k_read_ceiling (fdm_layer_read_ceiling): the same bytes per launch, "
                          "16-byte nontemporal loads, 64 KB per workgroup, no route / hand-off / math",
                "us_per_step": ceiling["us_per_step"],
                "kernel_avg_us": ceiling["kernel_avg_us"],
                "gbps": round(lb / (ceiling["kernel_avg_us"] * 1e-6) / 1e9, 1),
                "frac": round(lb / (ceiling["kernel_avg_us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                "layer_kernel_over_ceiling": round(k_us / ceiling["kernel_avg_us"], 3),
            },
        },
        "cpu_baseline": None,
    }
    if args.configs:
        result["matvec_q4k"] = bench_matvec(F, torch, args)
        result["expert_q4k_down"] = bench_expert(F, torch, "q4k")
        result["expert_q6k_down"] = bench_expert(F, torch, "q6k")
        result["layer_q6k_down"] = bench_layer_q6k(F, torch, args, stream, K)
    result["norm"] = bench_norm(F, torch, args, stream, K)
    if args.batched:
        result["batched"] = bench_batched(F, torch, layers, args, stream, K)
    if args.prefill:
        result["prefill"] = bench_prefill(F, torch, layers, args, stream, K)
    if args.dense:
        result["dense"] = bench_dense(F, torch, args, stream)
    if args.attn:
        result["attn"] = bench_attn(F, torch, args, stream, K=K)
    if args.stream:
        result["stream"] = bench_stream(F, torch, args, stream, K)
    if not args.no_cpu_baseline:
        ref, tuned = cpu_baseline(args.down, args.cpu_seconds, K)
        result["cpu_baseline"] = ref
        result["cpu_baseline_tuned"] = tuned
        result["speedup_vs_cpu"] = {"reference_shaped": round(ref["value"] / us_per_token, 1),
                                    "tuned_all_cores": round(tuned["value"] / us_per_token, 1)}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
