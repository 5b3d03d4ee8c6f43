"""Benchmark of the quantized-expert hot path on one MI355X.

Headline (`value`): MoE decode step of BASELINE config 2 -- batch 1, router
over 512 experts, top-10 + 1 shared expert, every expert a 4096->1024->4096
4-bit group-64 SwiGLU FFN -- in GB/s of algorithmic HBM traffic (the bytes of
every selected expert blob + x + h_mid + out).  A step = device routing
(softmax/top-K over fresh logits) + the fused expert step.  The pool holds all
512 experts (3.6 GB) and the shared expert rotates over 16 copies, so the
working set never fits the 256 MB MALL.

Also reported: prefill MoE-layer tokens/s (config 3) when built, the
per-kernel roofline of the fused decode launch pair measured with HIP events
on the launch stream, and a CPU baseline (the reference's own compiled
cpu_kernels.h matvec + SwiGLU, one host core) on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "flash-moe_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
H, I, E, K = 4096, 1024, 512, 10


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_pool(bits_of, seed):
    import numpy as np
    import fmoe_amd as fm
    from fmoe_amd import synth
    t = time.time()
    blobs = [synth.expert_blob((seed, e), H, I, bits_of(e)) for e in range(E)]
    pool = fm.DevicePool(blobs, [bits_of(e) for e in range(E)], H, I)
    log(f"pool of {E} experts generated + uploaded in {time.time() - t:.1f}s")
    sample = blobs[:K + 1]
    del blobs
    return pool, sample, np


def pmc_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE in KiB per dispatch, each scaled by what the counter reads for a plain
    device copy of known size); None when no summary exists."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    return round(d["fetch_kib"] * 1024 * d["fetch_scale"] + d["write_kib"] * 1024 * d["write_scale"])


def _decode_kernel_name(fused):
    """The kernel a one-token config-2 step runs: the row-split kernel where the
    library's switch enables it (FMOE_DECODE_BAL=1), else the per-CU item kernel."""
    bal = os.environ.get("FMOE_DECODE_BAL") == "1" and not os.environ.get("FMOE_DECODE_NO_BAL")
    tag = "true" if fused else "false"
    return f"fm_decode_bal_kernel<{tag}, false>" if bal else f"fm_decode_cu_kernel<16, {tag}>"


def graph_of(step, items):
    """step(i) for every i in items recorded into one HIP graph (on a side
    stream, as stream capture requires).  Replaying it runs exactly those
    kernels with no host work between them, as a serving loop would."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in items:
                step(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return g


def time_graph(g, n, warm=3):
    """ms per step of a graph of n steps, HIP events around one replay, after
    `warm` untimed replays (the first uploads the graph; the GPU's clocks settle
    over the next few milliseconds of sustained load)."""
    import torch
    for _ in range(max(1, warm)):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def bench_decode(args, dev):
    import numpy as np
    import torch
    import fmoe_amd as fm
    from fmoe_amd import synth

    pool, sample_blobs, _ = make_pool(lambda e: 4, 3000)
    args._pool = pool
    rng = synth.rng_for(3001)
    n_sh = 16
    shared_blobs = [synth.expert_blob((3002, i), H, I, 4) for i in range(n_sh)]
    sh_dev = [torch.from_numpy(b).to(dev) for b in shared_blobs]
    shared = [fm.experts_from_blob(d, 4, H, I) for d in sh_dev]
    nsteps = args.warmup + args.steps
    logits = torch.from_numpy(rng.normal(0, 1, (nsteps, E)).astype(np.float32)).to(dev)
    scores = torch.from_numpy(rng.normal(0, 1, nsteps).astype(np.float32)).to(dev)
    x = torch.from_numpy(synth.hidden_vec(rng, H)).to(dev)
    hm = torch.from_numpy(rng.normal(0, 1, H).astype(np.float32)).to(dev)
    idx = torch.empty((nsteps, K), dtype=torch.int32, device=dev)
    w = torch.empty((nsteps, K), dtype=torch.float32, device=dev)
    ws = fm.workspace(fm.decode_workspace_bytes(K + 1, H, I), dev)
    out = torch.empty(H, dtype=torch.float32, device=dev)
    ob = torch.empty(H, dtype=torch.int16, device=dev)

    def step(i):
        fm.route_topk(logits[i:i + 1], K, idx[i], w[i])
        fm.moe_decode_pool(pool, idx[i], w[i], x, out, ws, shared=shared[i % n_sh], shared_bits=4,
                           shared_score=scores[i:i + 1], h_mid=hm, out_bf16=ob)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # eager: one Python call per launch (host-bound at these kernel times)
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.warmup, nsteps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    eager_ms = e0.elapsed_time(e1) / args.steps
    # the timed steps: routing + fused step of every token, recorded into one
    # HIP graph (the kernels keep their hand-off tag on the device, so replays
    # are valid) and replayed back to back
    g = graph_of(step, range(args.warmup, nsteps))
    step_ms = time_graph(g, args.steps)
    status = fm.workspace_status(ws)
    if status:
        raise SystemExit(f"decode workspace status {status}: a step's output is invalid")
    del g
    # the same steps through fm_moe_route_decode_pool: routing fused into the
    # step's launch (one kernel per step); its routing must equal the routing
    # kernel's bit for bit
    idx_f = torch.empty_like(idx)
    w_f = torch.empty_like(w)

    def step_fused(i):
        fm.moe_route_decode_pool(pool, logits[i], idx_f[i], w_f[i], x, out, ws, shared=shared[i % n_sh],
                                 shared_bits=4, shared_score=scores[i:i + 1], h_mid=hm, out_bf16=ob)

    for i in range(args.warmup):
        step_fused(i)
    g = graph_of(step_fused, range(args.warmup, nsteps))
    fused_ms = time_graph(g, args.steps)
    del g
    status = fm.workspace_status(ws)
    if status:
        raise SystemExit(f"decode workspace status {status}: a fused step's output is invalid")
    if not (torch.equal(idx_f[args.warmup:], idx[args.warmup:]) and torch.equal(w_f[args.warmup:], w[args.warmup:])):
        raise SystemExit("fused routing differs from fm_route_topk")
    # algorithmic bytes per step: K routed + shared blobs, x, h_mid, out fp32 + bf16
    blob = fm.layout_of(H, I, 64, 4).size
    step_bytes = (K + 1) * blob + H * 4 * 3 + H * 2 + E * 4
    # the fused expert kernel alone: back-to-back launches (routing already
    # done above for every step) between two events on its stream
    torch.cuda.synchronize()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def dec(i):
        fm.moe_decode_pool(pool, idx[i], w[i], x, out, ws, shared=shared[i % n_sh], shared_bits=4,
                           shared_score=scores[i:i + 1], h_mid=hm, out_bf16=ob)

    g = graph_of(dec, range(args.warmup, nsteps))
    kern_ms = time_graph(g, args.steps)
    del g
    # the same launches with the next layer's input RMS norm fused into the combine
    nw = torch.from_numpy(synth.bf16_bits(rng.normal(1, 0.1, H).astype(np.float32)).view(np.int16)).to(dev)
    normed = torch.empty(H, dtype=torch.float32, device=dev)
    def dec_norm(i):
        fm.moe_decode_pool_norm(pool, idx[i], w[i], x, out, ws, nw, 1e-6, normed, shared=shared[i % n_sh],
                                shared_bits=4, shared_score=scores[i:i + 1], h_mid=hm, out_bf16=ob)

    g = graph_of(dec_norm, range(args.warmup, nsteps))
    norm_ms = time_graph(g, args.steps)
    del g
    # the whole MoE block of one decode token through the C layer driver
    # (fm_moe_forward): router + shared-gate matvecs, routing, fused experts
    Wr, sr, br = synth.quant_matrix(synth.rng_for(3010), E, H, 4)
    Wg, sgt, bgt = synth.quant_matrix(synth.rng_for(3011), 1, H, 4)
    dl = [torch.from_numpy(np.ascontiguousarray(t)).to(dev) for t in (Wr, sr, br, Wg, sgt, bgt)]
    Lr = fm.MoeLayer()
    Lr.router_w, Lr.router_s, Lr.router_b = dl[0].data_ptr(), dl[1].data_ptr(), dl[2].data_ptr()
    Lr.router_bits = 4
    Lr.seg_w, Lr.seg_s, Lr.seg_b = dl[3].data_ptr(), dl[4].data_ptr(), dl[5].data_ptr()
    Lr.seg_bits = 4
    Lr.shared_bits = 4
    Lr.has_shared = 1
    Lr.pool = pool.c
    lws = fm.workspace(fm.moe_forward_workspace_bytes(Lr, K), dev)
    hps = torch.from_numpy(synth.hidden_vec(rng, H, (16, H))).to(dev)
    def layer(i):
        Lr.shared = shared[i % n_sh]
        fm.moe_forward(Lr, K, hps[i % 16], hm, out, lws, out_bf16=ob)

    for i in range(args.warmup):
        layer(i)
    g = graph_of(layer, range(args.steps))
    layer_ms = time_graph(g, args.steps)
    del g
    router_bytes = E * H // 2 + E * (H // 64) * 4 + H // 2 + (H // 64) * 4
    kern_bytes = (K + 1) * blob + H * 4 * 3 + H * 2
    # unique experts actually touched per step (routing may repeat across steps, never within)
    achieved = kern_bytes / (kern_ms * 1e-3) / 1e9
    # the headline step is ONE launch of the fused kernel (routing + experts):
    # its algorithmic bytes are the step's plus the K routing outputs
    fused_bytes = step_bytes + K * 8
    fused_gbs = fused_bytes / (fused_ms * 1e-3) / 1e9
    res = {
        "step_ms": fused_ms, "two_launch_step_ms": step_ms, "wall_s": wall, "step_bytes": step_bytes, "eager_us_per_step": round(eager_ms * 1e3, 2),
        "value": step_bytes / (fused_ms * 1e-3) / 1e9,
        "roofline": {"bound": "hbm", "achieved": fused_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": fused_gbs / HBM_PEAK_GBS, "traffic": pmc_traffic("decode_fused_config2_pmc.json"),
                     "kernel": _decode_kernel_name(True) + " (one fm_moe_route_decode_pool call: routing + experts)",
                     "kernel_us": fused_ms * 1e3, "bytes_per_launch": fused_bytes,
                     "decode_only": {"kernel": _decode_kernel_name(False) + " (one fm_moe_decode_pool call, "
                                               "routing done by fm_route_kernel)",
                                     "kernel_us": kern_ms * 1e3, "bytes_per_launch": kern_bytes,
                                     "achieved": achieved, "frac": achieved / HBM_PEAK_GBS,
                                     "traffic": pmc_traffic("decode_config2_pmc.json"),
                                     "kernel_us_with_fused_rms_norm": norm_ms * 1e3}},
        "layer_step": {"path": "fm_moe_forward: router + shared-gate matvecs (4-bit) -> routing fused into the expert step",
                       "us": round(layer_ms * 1e3, 2), "bytes": kern_bytes + router_bytes,
                       "gbs": round((kern_bytes + router_bytes) / (layer_ms * 1e-3) / 1e9, 1)},
    }
    return res, sample_blobs


def bench_qwen35(args, dev):
    """The reference's other model shape (Qwen3.5-35B-A3B: hidden 2048,
    moe_intermediate 512, 256 experts, K = 8 + a shared expert of 512):
    decode step (routing + fused experts) as a HIP graph, and the kernel alone."""
    import numpy as np
    import torch
    import fmoe_amd as fm
    from fmoe_amd import synth
    h, i_, e_, k_ = 2048, 512, 256, 8
    blobs = [synth.expert_blob((3500, e), h, i_, 4) for e in range(e_)]
    pool = fm.DevicePool(blobs, [4] * e_, h, i_)
    del blobs
    sh_dev = [torch.from_numpy(synth.expert_blob((3501, j), h, i_, 4)).to(dev) for j in range(16)]
    shared = [fm.experts_from_blob(d, 4, h, i_) for d in sh_dev]
    rng = synth.rng_for(3502)
    nsteps = args.warmup + args.steps
    logits = torch.from_numpy(rng.normal(0, 1, (nsteps, e_)).astype(np.float32)).to(dev)
    scores = torch.from_numpy(rng.normal(0, 1, nsteps).astype(np.float32)).to(dev)
    x = torch.from_numpy(synth.hidden_vec(rng, h)).to(dev)
    hm = torch.from_numpy(rng.normal(0, 1, h).astype(np.float32)).to(dev)
    idx = torch.empty((nsteps, k_), dtype=torch.int32, device=dev)
    w = torch.empty((nsteps, k_), dtype=torch.float32, device=dev)
    ws = fm.workspace(fm.decode_workspace_bytes(k_ + 1, h, i_), dev)
    out = torch.empty(h, dtype=torch.float32, device=dev)

    def dec(j):
        fm.moe_decode_pool(pool, idx[j], w[j], x, out, ws, shared=shared[j % 16], shared_bits=4,
                           shared_score=scores[j:j + 1], h_mid=hm)

    def step2(j):
        fm.route_topk(logits[j:j + 1], k_, idx[j], w[j])
        dec(j)

    def step(j):  # routing fused into the step's launch
        fm.moe_route_decode_pool(pool, logits[j], idx[j], w[j], x, out, ws, shared=shared[j % 16], shared_bits=4,
                                 shared_score=scores[j:j + 1], h_mid=hm)

    for j in range(args.warmup):
        step2(j)
        step(j)
    g = graph_of(step2, range(args.warmup, nsteps))
    step2_ms = time_graph(g, args.steps)
    del g
    g = graph_of(step, range(args.warmup, nsteps))
    step_ms = time_graph(g, args.steps)
    del g
    g = graph_of(dec, range(args.warmup, nsteps))
    kern_ms = time_graph(g, args.steps)
    del g
    if fm.workspace_status(ws):
        raise SystemExit("qwen3.5-35b decode: workspace status set")
    nbytes = (k_ + 1) * fm.layout_of(h, i_, 64, 4).size + h * 4 * 3
    return {"workload": "Qwen3.5-35B-A3B shape: hidden 2048, inter 512, 256 experts, top-8 + shared, 4-bit",
            "step_us": round(step_ms * 1e3, 2), "path": "fm_moe_route_decode_pool (one launch)",
            "two_launch_step_us": round(step2_ms * 1e3, 2), "kernel_us": round(kern_ms * 1e3, 2), "bytes": nbytes,
            "kernel_gbs": round(nbytes / kern_ms / 1e6, 1), "kernel_hbm_frac": round(nbytes / kern_ms / 1e6 / HBM_PEAK_GBS, 4)}


def bench_prefill(args, dev, pool):
    """Config 3: 512 tokens, 512 experts, top-10 over Zipf(1.1) logits + shared
    expert, one MoE layer = routing + grouped expert GEMMs + combine."""
    import numpy as np
    import torch
    import fmoe_amd as fm
    from fmoe_amd import synth
    Tn = 512
    rng = synth.rng_for(3101)
    n = args.prefill_warmup + args.prefill_steps
    logits = [torch.from_numpy(synth.zipf_logits(rng, Tn, E)).to(dev) for _ in range(n)]
    X = torch.from_numpy(synth.hidden_vec(rng, H, (Tn, H))).to(dev)
    hm = torch.from_numpy(rng.normal(0, 1, (Tn, H)).astype(np.float32)).to(dev)
    g = torch.from_numpy(rng.normal(0, 1, Tn).astype(np.float32)).to(dev)
    sh_blob = torch.from_numpy(synth.expert_blob((3102, 0), H, I, 4)).to(dev)
    sh = fm.experts_from_blob(sh_blob, 4, H, I)
    idx = torch.empty((Tn, K), dtype=torch.int32, device=dev)
    w = torch.empty((Tn, K), dtype=torch.float32, device=dev)
    ws = fm.workspace(fm.prefill_workspace_bytes(Tn, K, pool), dev)
    out = torch.empty((Tn, H), dtype=torch.float32, device=dev)
    ob = torch.empty((Tn, H), dtype=torch.int16, device=dev)

    def step(i):
        fm.route_topk(logits[i], K, idx, w)
        fm.prefill_moe(pool, idx, w, X, out, ws, shared=sh, shared_bits=4, shared_scores=g, h_mid=hm, out_bf16=ob)

    uniq = []
    for i in range(args.prefill_warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.prefill_warmup, n):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.prefill_steps
    for i in range(args.prefill_warmup, n):
        fm.route_topk(logits[i], K, idx, w)
        uniq.append(len(np.unique(idx.cpu().numpy())))
    blob = fm.layout_of(H, I, 64, 4).size
    bytes_step = (float(np.mean(uniq)) + 1) * blob + Tn * H * 4 * 3 + Tn * H * 2
    flops = (Tn * K + Tn) * 3 * 2 * H * I
    return {"ms": ms, "tokens_per_s": Tn / (ms * 1e-3), "unique_experts": float(np.mean(uniq)),
            "hbm_gbs": bytes_step / (ms * 1e-3) / 1e9, "hbm_frac": bytes_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "tflops": flops / (ms * 1e-3) / 1e12, "mfma_frac": flops / (ms * 1e-3) / 2.5e15,
            "bytes_per_step": bytes_step, "flops_per_step": flops}


def bench_tiered(args, dev):
    """Config 4: the config-2 layer with 128 hot 4-bit experts (seeded
    permutation) and 384 cold 2-bit ones; decode at batch 1 (route + fused
    step) and batch 4 (route 4 tokens + grouped expert kernel over the union of
    their experts).  Bytes = unique selected blobs + shared + activations."""
    import numpy as np
    import torch
    import fmoe_amd as fm
    from fmoe_amd import synth
    perm = synth.rng_for(3201).permutation(E)
    hot = set(int(e) for e in perm[:128])
    bits_of = lambda e: 4 if e in hot else 2  # noqa: E731
    pool, _, _ = make_pool(bits_of, 3200)
    rng = synth.rng_for(3202)
    sizes = {b: fm.layout_of(H, I, 64, b).size for b in (2, 4)}
    sh_blob = torch.from_numpy(synth.expert_blob((3203, 0), H, I, 4)).to(dev)
    sh = fm.experts_from_blob(sh_blob, 4, H, I)
    res = {}
    for B in (1, 4):
        n = args.warmup + args.steps
        logits = torch.from_numpy(rng.normal(0, 1, (n, B, E)).astype(np.float32)).to(dev)
        scores = torch.from_numpy(rng.normal(0, 1, (n, B)).astype(np.float32)).to(dev)
        X = torch.from_numpy(synth.hidden_vec(rng, H, (B, H))).to(dev)
        hm = torch.from_numpy(rng.normal(0, 1, (B, H)).astype(np.float32)).to(dev)
        idx = torch.empty((n, B, K), dtype=torch.int32, device=dev)
        w = torch.empty((n, B, K), dtype=torch.float32, device=dev)
        out = torch.empty((B, H), dtype=torch.float32, device=dev)
        ob = torch.empty((B, H), dtype=torch.int16, device=dev)
        if B == 1:
            ws = fm.workspace(fm.decode_workspace_bytes(K + 1, H, I), dev)
        else:
            ws = fm.workspace(fm.prefill_workspace_bytes(B, K, pool), dev)

        def step(i):
            if B == 1:  # routing fused into the step's launch
                fm.moe_route_decode_pool(pool, logits[i, 0], idx[i, 0], w[i, 0], X[0], out[0], ws, shared=sh,
                                         shared_bits=4, shared_score=scores[i, :1], h_mid=hm[0], out_bf16=ob[0])
            else:
                fm.route_topk(logits[i], K, idx[i], w[i])
                fm.prefill_moe(pool, idx[i], w[i], X, out, ws, shared=sh, shared_bits=4, shared_scores=scores[i],
                               h_mid=hm, out_bf16=ob)

        for i in range(args.warmup):
            step(i)
        g = graph_of(step, range(args.warmup, n))
        ms = time_graph(g, args.steps)
        del g
        ids = idx[args.warmup:].cpu().numpy()
        nbytes = []
        for i in range(args.steps):
            u = np.unique(ids[i])
            nbytes.append(sum(sizes[bits_of(int(e))] for e in u) + sizes[4] + B * H * (4 * 3 + 2))
        step_bytes = float(np.mean(nbytes))
        res[f"b{B}"] = {"us_per_step": ms * 1e3, "bytes_per_step": round(step_bytes),
                        "gbs": step_bytes / (ms * 1e-3) / 1e9,
                        "hbm_frac": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                        "path": "fm_moe_route_decode_pool (one launch)" if B == 1 else "route + fm_prefill_moe (few tokens: all tokens' slots in one multi-pass decode launch)"}
    del pool
    return res


def bench_small(args, dev, pool):
    """Configs 0 and 1: one 4096x4096 4-bit matvec (fm_dequant_matvec) and one
    SwiGLU expert scaled by a router weight (fm_moe_decode, K = 1), back-to-back
    launches rotating over more weights than the 256 MB MALL holds (32 matrix
    copies; the 512-expert pool)."""
    import numpy as np
    import torch
    import fmoe_amd as fm
    from fmoe_amd import synth
    n = 32
    W, sc, bi = synth.quant_matrix(synth.rng_for(3300), 4096, 4096, 4)
    dW = torch.from_numpy(W).to(dev)
    ds = torch.from_numpy(sc.view(np.int16)).to(dev)
    db = torch.from_numpy(bi.view(np.int16)).to(dev)
    copies = [(dW.clone(), ds.clone(), db.clone()) for _ in range(n)]
    x = torch.from_numpy(synth.hidden_vec(synth.rng_for(3301), 4096)).to(dev)
    y = torch.empty(4096, dtype=torch.float32, device=dev)
    steps = max(args.steps, 100)
    # arguments built once and the C entry points called directly, so the
    # launches outpace the GPU (a Python wrapper per call would not)
    import ctypes
    L = fm.lib()
    mv_args = [(c[0].data_ptr(), c[1].data_ptr(), c[2].data_ptr()) for c in copies]
    xp, yp = x.data_ptr(), y.data_ptr()

    def mv(i):
        w_, s_, b_ = mv_args[i % n]
        return L.fm_dequant_matvec(w_, s_, b_, xp, yp, 4096, 4096, 64, 4, fm.stream_ptr())

    for i in range(10):
        fm.check(mv(i))
    g = graph_of(mv, range(steps))
    mv_us = time_graph(g, steps) * 1e3
    del g
    mv_bytes = 4096 * 512 * 4 + 2 * 4096 * 64 * 2 + 4096 * 2 + 4096 * 4
    ws = fm.workspace(fm.decode_workspace_bytes(1, H, I), dev)
    out = torch.empty(H, dtype=torch.float32, device=dev)
    ex_args = []
    for e in range(E):
        arr = (fm.ExpertWeights * 1)(pool.expert(e))
        ex_args.append(arr)
    bits1, w1 = (ctypes.c_int * 1)(4), (ctypes.c_float * 1)(0.37)
    wsp, wsb, outp = ws.data_ptr(), ws.numel(), out.data_ptr()

    def ex(i):
        return L.fm_moe_decode(1, ex_args[(i * 37) % E], bits1, w1, None, None, 4, 0, 0.0, H, I, 64, xp, None, outp,
                               None, wsp, wsb, fm.stream_ptr())

    for i in range(10):
        fm.check(ex(i))
    g = graph_of(ex, range(steps))
    ex_us = time_graph(g, steps) * 1e3
    del g
    ex_bytes = fm.layout_of(H, I, 64, 4).size + H * 2 + H * 4
    return {"config0_matvec": {"workload": "4096x4096 4-bit g64 matvec, 32 rotating copies", "us": round(mv_us, 2),
                               "bytes": mv_bytes, "gbs": round(mv_bytes / mv_us / 1e3, 1),
                               "hbm_frac": round(mv_bytes / mv_us / 1e3 / HBM_PEAK_GBS, 4)},
            "config1_expert": {"workload": "one 4096->1024->4096 4-bit SwiGLU expert x router weight, 512 rotating",
                               "us": round(ex_us, 2), "bytes": ex_bytes, "gbs": round(ex_bytes / ex_us / 1e3, 1),
                               "hbm_frac": round(ex_bytes / ex_us / 1e3 / HBM_PEAK_GBS, 4)}}


def bench_staging(args, dev):
    """Expert files -> HBM (fm_expert_io.h), from a warm page cache: a whole layer
    file loaded into device memory, and per-token staging of K+1 experts
    (pread into pinned buffers + host->device copies), the reference's
    async_pread_start/wait step (expert_io.h:183-266).  Bounded by PCIe, not HBM."""
    import shutil
    import tempfile
    import numpy as np
    import torch
    import fmoe_amd as fm
    from fmoe_amd.expert_io import STORE_4BIT, ExpertStore
    ne = 64
    s4 = fm.layout_of(H, I, 64, 4).size
    d = tempfile.mkdtemp(prefix="fm_stage_")
    try:
        os.makedirs(os.path.join(d, "packed_experts"))
        rng = np.random.default_rng(5)
        with open(os.path.join(d, "packed_experts", "layer_00.bin"), "wb") as f:
            for _ in range(ne):
                f.write(rng.integers(0, 256, s4, dtype=np.uint8).tobytes())
        # 4 workers: more parallel page-cache copies compete with the DMA for host memory
        with ExpertStore(d, 1, ne, H, I, mode=STORE_4BIT, io_threads=4) as st:
            times = []
            for _ in range(3):
                torch.cuda.synchronize()
                t = time.perf_counter()
                lp = st.load_layer(0)
                times.append(time.perf_counter() - t)
                del lp
            load_gbs = ne * s4 / min(times) / 1e9
            bufs = torch.empty((2, K + 1, s4), dtype=torch.uint8, device=dev)
            ptrs = [[bufs[j, k].data_ptr() for k in range(K + 1)] for j in range(2)]
            steps = 60
            ids = [[int(e) for e in rng.permutation(ne)[:K + 1]] for _ in range(steps)]
            for i in range(5):
                st.stage(0, ids[i], ptrs[i & 1])
            torch.cuda.synchronize()
            t = time.perf_counter()
            for i in range(steps):  # latency: each token's experts in HBM before the next starts
                st.stage(0, ids[i], ptrs[i & 1])
                torch.cuda.synchronize()
            dt = (time.perf_counter() - t) / steps
            t = time.perf_counter()
            for i in range(steps):  # pipelined: reads of token i+1 overlap the copies of token i
                st.stage(0, ids[i], ptrs[i & 1])
            torch.cuda.synchronize()
            dp = (time.perf_counter() - t) / steps
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return {"workload": f"{ne} 4-bit experts in packed_experts/layer_00.bin (page cache warm); "
                        f"per-token staging of {K + 1} experts", "layer_load_gbs": round(load_gbs, 2),
            "stage_us_per_token": round(dt * 1e6, 1), "stage_gbs": round((K + 1) * s4 / dt / 1e9, 2),
            "stage_pipelined_us_per_token": round(dp * 1e6, 1),
            "stage_pipelined_gbs": round((K + 1) * s4 / dp / 1e9, 2), "io_threads": 4,
            "bound": "host pread + PCIe host->device copy"}


def host_info():
    """CPU model and the cores this process may use (the box's host, not the GPU)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count()}


def cpu_baseline(budget_s=10.0):
    """The reference's own CPU path (oracle/_ref: cpu_dequant_matvec, cpu_swiglu,
    cpu_vec_madd compiled from cpu_kernels.h; one core, as the reference runs
    it) on bounded samples of configs 0-4.  Weights rotate over ~700 MB of
    distinct blobs so the host's last-level cache cannot hold them.  Config 4's
    2-bit experts use this build's C port (the reference has no CPU 2-bit kernel:
    its CPU fallback misreads 2-bit blobs with the 4-bit kernel,
    layer_forward.h:4106-4129)."""
    import numpy as np
    from fmoe_amd import synth
    from fmoe_amd.layout import expert_offsets
    kind = "reference"
    try:
        from oracle import RefLib
        R = RefLib()
    except Exception:
        R = None
        kind = "port"
    from oracle import OracleLib
    O = OracleLib()
    per = budget_s / 5.0
    t_gen = time.perf_counter()
    NB = 96
    blobs4 = [synth.expert_blob((3400, e), H, I, 4) for e in range(NB)]
    blobs2 = [synth.expert_blob((3401, e), H, I, 2) for e in range(48)]
    gen_s = time.perf_counter() - t_gen
    off4, size4 = expert_offsets(H, I, 64, 4)
    size2 = expert_offsets(H, I, 64, 2)[1]
    x = synth.hidden_vec(synth.rng_for(5), H)

    def mats(blob, name, rows, cols):
        w = blob[off4[name + "_w"]: off4[name + "_w"] + rows * cols // 2].view(np.uint32).reshape(rows, cols // 8)
        s = blob[off4[name + "_s"]: off4[name + "_s"] + rows * cols // 32].view(np.uint16).reshape(rows, -1)
        b = blob[off4[name + "_b"]: off4[name + "_b"] + rows * cols // 32].view(np.uint16).reshape(rows, -1)
        return w, s, b

    def expert(blob, bits, xin):
        if R is None or bits == 2:
            return O.expert_forward(blob, bits, H, I, xin)
        g = R.matvec4(*mats(blob, "gate", I, H), xin)
        u = R.matvec4(*mats(blob, "up", I, H), xin)
        return R.matvec4(*mats(blob, "down", H, I), R.swiglu(g, u))

    def madd(acc, e, w):
        return R.vec_madd(acc, e, w) if R is not None else acc + np.float32(w) * e

    def timed(fn):
        n, t0 = 0, time.perf_counter()
        while True:
            fn(n)
            n += 1
            if time.perf_counter() - t0 > per:
                return n, time.perf_counter() - t0

    res = {}
    # config 0: 4096 x 4096 matvec; W views into the blob bytes (any byte is a
    # valid pair of codes), real scales/biases
    big = np.concatenate(blobs4[:40])
    _, s0, b0 = synth.quant_matrix(synth.rng_for(3402), 4096, 4096, 4)
    mv_w = 4096 * 512 * 4
    nw = big.size // mv_w
    Ws = [big[i * mv_w:(i + 1) * mv_w].view(np.uint32).reshape(4096, 512) for i in range(nw)]
    mv = (lambda W: R.matvec4(W, s0, b0, x)) if R is not None else (lambda W: O.matvec(4, W, s0, b0, x))
    n, dt = timed(lambda i: mv(Ws[i % nw]))
    mv_bytes = 4096 * 512 * 4 + 2 * 4096 * 64 * 2
    res["config0_matvec"] = {"us": round(dt / n * 1e6, 1), "gbs": round(mv_bytes * n / dt / 1e9, 3),
                             "sample": f"{n} matvecs over {nw} distinct 8 MB matrices"}
    del big, Ws
    # config 1: one expert x router weight
    n, dt = timed(lambda i: expert(blobs4[(i * 7) % NB], 4, x))
    res["config1_expert"] = {"us": round(dt / n * 1e6, 1), "gbs": round(size4 * n / dt / 1e9, 3),
                             "sample": f"{n} expert forwards over {NB} blobs"}
    # config 2: decode step, 10 routed + shared, weighted sum (cpu_vec_madd)
    w10 = np.full(K, 0.1, np.float32)

    def step(i, xin=x):
        acc = np.zeros(H, np.float32)
        for k in range(K):
            acc = madd(acc, expert(blobs4[(i * 11 + k) % NB], 4, xin), w10[k])
        return madd(acc, expert(blobs4[(i * 11 + K) % NB], 4, xin), 0.5)

    n, dt = timed(step)
    res["config2_decode"] = {"us_per_step": round(dt / n * 1e6, 1), "gbs": round((K + 1) * size4 * n / dt / 1e9, 3),
                             "sample": f"{n} decode steps (11 4-bit experts each) over {NB} blobs"}
    # config 3: prefill as the reference runs routed experts -- per token
    # (batched_prefill.h:241-308): tokens/s of the same per-token work
    X = synth.hidden_vec(synth.rng_for(6), H, (16, H))
    n, dt = timed(lambda i: step(i, X[i % 16]))
    res["config3_prefill"] = {"tokens_per_s": round(n / dt, 2), "ms_per_token": round(dt / n * 1e3, 2),
                              "sample": f"{n} tokens x 11 expert forwards (per-token, as batched_prefill.h "
                                        f"runs routed experts)"}
    # config 4: tiered decode b=1 (about a quarter of the routed experts 4-bit)
    def tstep(i):
        acc = np.zeros(H, np.float32)
        for k in range(K):
            j = i * 11 + k
            e = expert(blobs4[j % NB], 4, x) if j % 4 == 0 else expert(blobs2[j % 48], 2, x)
            acc = madd(acc, e, w10[k])
        return madd(acc, expert(blobs4[(i * 11 + K) % NB], 4, x), 0.5)

    n, dt = timed(tstep)
    nbytes = sum(size4 if (i * 11 + k) % 4 == 0 else size2 for i in range(1) for k in range(K)) + size4
    res["config4_tiered_b1"] = {"us_per_step": round(dt / n * 1e6, 1), "gbs": round(nbytes * n / dt / 1e9, 3),
                                "sample": f"{n} tiered decode steps (2-bit experts: C port)"}
    c2 = res["config2_decode"]
    return {"value": c2["gbs"], "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": c2["sample"] + f"; {per:.1f} s per config, blobs generated in {gen_s:.1f} s",
            "host": host_info(), "configs": res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work (5 configs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--prefill-warmup", type=int, default=30,
                    help="untimed layers first: the GPU's clocks take ~20 ms of sustained load to settle")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-tiered", action="store_true")
    ap.add_argument("--no-staging", action="store_true")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run 10 device copies of MIB MiB (scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import fmoe_amd as fm
    fm.lib()
    dev = torch.device("cuda:0")
    if args.copy_calib:
        src = torch.empty(args.copy_calib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: 10 x {args.copy_calib} MiB")
        return
    dec, sample = bench_decode(args, dev)
    log(f"decode: {dec['step_ms'] * 1e3:.2f} us/step, {dec['value']:.0f} GB/s; decode-only launch "
        f"{dec['roofline']['decode_only']['kernel_us']:.2f} us = {dec['roofline']['decode_only']['achieved']:.0f} GB/s; "
        f"whole MoE block "
        f"(router + routing + experts) {dec['layer_step']['us']} us")
    small = bench_small(args, dev, args._pool)
    log(f"config 0 matvec: {small['config0_matvec']['us']} us = {small['config0_matvec']['gbs']} GB/s; "
        f"config 1 expert: {small['config1_expert']['us']} us = {small['config1_expert']['gbs']} GB/s")
    q35 = bench_qwen35(args, dev)
    log(f"qwen3.5-35b shape: step {q35['step_us']} us, kernel {q35['kernel_us']} us = {q35['kernel_gbs']} GB/s")
    pre = None if args.no_prefill else bench_prefill(args, dev, args._pool)
    if pre:
        log(f"prefill: {pre['ms']:.3f} ms/layer, {pre['tokens_per_s']:.0f} tok/s, {pre['hbm_gbs']:.0f} GB/s, "
            f"{pre['tflops']:.1f} TFLOP/s")
    tiered = None if args.no_tiered else bench_tiered(args, dev)
    if tiered:
        for k, v in tiered.items():
            log(f"tiered {k}: {v['us_per_step']:.2f} us/step, {v['gbs']:.0f} GB/s ({v['path']})")
    staging = None if args.no_staging else bench_staging(args, dev)
    if staging:
        log(f"staging: layer load {staging['layer_load_gbs']} GB/s; per token {staging['stage_us_per_token']} us "
            f"= {staging['stage_gbs']} GB/s; pipelined {staging['stage_pipelined_gbs']} GB/s")
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_budget)
    line = {
        "metric": "4-bit expert FFN decode GB/s (% of HBM peak); prefill MoE-layer tokens/s",
        "value": round(dec["value"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": dec["step_ms"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4 codes x f16 -> f32 accumulate", "data": "synthetic (seeded, random-init)",
        "hbm_frac": dec["value"] / HBM_PEAK_GBS,
        "config": {"workload": "config 2: MoE decode b=1, 512 experts, top-10 + shared, "
                               "4096->1024->4096 SwiGLU, 4-bit g64, device routing",
                   "experts_per_step": K + 1, "bytes_per_step": dec["step_bytes"],
                   "path": "fm_moe_route_decode_pool (routing fused into the step: one launch per step)",
                   "timing": "the K timed steps recorded into one HIP graph, replayed once between HIP events "
                             "after three untimed replays of it",
                   "two_launch_us_per_step": round(dec["two_launch_step_ms"] * 1e3, 2),
                   "eager_us_per_step": dec["eager_us_per_step"]},
        "roofline": dec["roofline"],
        "layer_step": dec["layer_step"],
        "single": small,
        "qwen35_shape": q35,
        "prefill": None if pre is None else {
            "workload": "config 3: 512 tokens, 512 experts, top-10 Zipf(1.1) + shared, grouped MFMA dequant-GEMM",
            "tokens_per_s": round(pre["tokens_per_s"]), "ms_per_layer": pre["ms"],
            "unique_experts": pre["unique_experts"], "hbm_gbs": round(pre["hbm_gbs"], 1),
            "hbm_frac": pre["hbm_frac"], "tflops": round(pre["tflops"], 2), "mfma_frac": pre["mfma_frac"]},
        "tiered": None if tiered is None else {
            "workload": "config 4: config-2 layer with 128 hot 4-bit + 384 cold 2-bit experts, "
                        "top-10 + 4-bit shared, batch 1 and 4", **{k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                                                                  for kk, vv in v.items()} for k, v in tiered.items()}},
        "staging": staging,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
