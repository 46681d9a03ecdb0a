#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X (BASELINE.json metric: MoE-layer tokens/s at M=1 and
M=512, with achieved HBM GB/s against the 8 TB/s roofline).

A step is one MoE layer call (router -> top-k -> dispatch -> Q4_K SwiGLU experts + shared expert
-> combine) over one batch of M synthetic tokens.  Steps rotate through a stack of --layers
distinct layers (48 = BASELINE config 5, ~43.5 GB of Q4_K experts resident in HBM) so that the
256 MB Infinity Cache cannot serve repeats.  Weights and inputs are generated on the GPU
(random-init Q4_K superblocks of the configs' shapes) and are resident before timing starts.

Prints ONE JSON line.  `value` is the M=1 decode layer rate; the other M
(configs 2 and 3) are reported under "results", with config 4 (M=3072, Q6_K down projections,
dynamic-k routing) and config 5 (the 48-layer RMSNorm + residual stack, timed end to end at M=1
and M=512).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tr-infer_amd"))

H, E, F, K = 2048, 512, 512, 10
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
Q4K_ROW_H = H // 256 * 144   # bytes of a gate/up row (K = H)
Q4K_ROW_F = F // 256 * 144   # bytes of a down row (K = F)
EXPERT_BYTES = 2 * F * Q4K_ROW_H + H * Q4K_ROW_F   # 1,769,472


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_bytes(n_experts_touched, M):
    """Algorithmic HBM bytes of one layer call (each byte counted once): touched experts, the
    shared expert, the f32 router, the shared gate vector, x in and out in f32."""
    return n_experts_touched * EXPERT_BYTES + EXPERT_BYTES + E * H * 4 + H * 4 + M * H * 4 * 2


def layer_ops(n_ent, M):
    return (n_ent + M) * 3 * 2 * H * F


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--m", type=str, default="1,4,8,16,512")
    ap.add_argument("--extra", type=str, default="c4,stack,tq,hc,gemv",
                    help="also time config 4 (c4: M=3072, Q6_K down, dynamic-k) and config 5 (stack: the "
                         "48-layer RMSNorm + residual stack at M=1 and M=512); tq: the layer on packed TQ "
                         "experts at the real shape (H=2560, F=640) at M=1, 4 and 512; hc: the same layer "
                         "behind the hyper-connection mix (trk_moe_forward_hc, hc=4, low rank 320); gemv: "
                         "trk_gemv on the real model's dense projections; q80 / q51 / q6k: the layer at M=1 "
                         "and M=512 with Q8_0 / Q5_1 / Q6_K downs; '' for none")
    ap.add_argument("--tq-layers", type=int, default=24,
                    help="layers in the rotation of the TQ extra (1.78 GB of experts each)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph replay")
    ap.add_argument("--fusion", type=int, default=None, choices=(0, 1),
                    help="force the one-launch decode layer on (1) or off (0); default: the library's choice")
    ap.add_argument("--stream-rows", type=int, default=None, metavar="ROWS",
                    help="batch items of at most ROWS rows on the streaming GEMV (-1 the library's choice, "
                         "0 all on the MFMA tiles)")
    ap.add_argument("--decode-rows", type=int, default=None, metavar="ROWS",
                    help="batches of 2..ROWS tokens as per-token decode units (0 never; default: the "
                         "library's, 8)")
    ap.add_argument("--copy-cal", type=int, default=0, metavar="MIB",
                    help="finish with three device copies of MIB MiB (a known-size kernel for calibrating "
                         "rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU: the MoE block on one MI355X; "
                                   "multi-GPU sharding is not built (expert parallelism over RCCL is a "
                                   "design only)", "n_gpus": args.gpus}))
        sys.exit(2)

    import numpy as np
    import torch
    import trmoe

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream()
    ms_list = [int(v) for v in args.m.split(",")]
    m_max = max(ms_list)

    t0 = time.time()
    bias = torch.from_numpy(trmoe.zipf_bias(1, E)).to(dev)
    layers = [trmoe.LayerWeights.generate(1, l, H, E, F, device=dev) for l in range(args.layers)]
    torch.cuda.synchronize()
    log(f"generated {args.layers} layers ({args.layers * E * EXPERT_BYTES / 1e9:.1f} GB experts) in {time.time() - t0:.1f}s")
    ctx = trmoe.Context(H, E, F, K, m_max)
    if args.fusion is not None:
        ctx.set_fusion(args.fusion)
    if args.stream_rows is not None:
        ctx.set_stream_rows(args.stream_rows)
    if args.decode_rows is not None:
        ctx.set_decode_rows(args.decode_rows)
    xs = {M: trmoe.gen_normal(1, (9 << 32) | M, M * H, 1.0, device=dev).view(M, H) for M in ms_list}
    out = torch.empty((m_max, H), dtype=torch.float32, device=dev)

    def weights(l, M):
        w = layers[l]
        # config 3 and larger batches: Zipf-skewed routing through an additive router bias
        w.moew.router_bias = bias.data_ptr() if M >= 512 else None
        return w

    results = {}
    for M in ms_list:
        x = xs[M]
        # pre-pass: the experts each layer touches for this input (for the algorithmic bytes)
        touched, ents, maxg = [], [], []
        for l in range(args.layers):
            ctx.forward(weights(l, M), x, out[:M])
            ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
            nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
            sel = np.concatenate([ids[t, :nsel[t]] for t in range(M)])
            touched.append(len(np.unique(sel)))
            ents.append(int(nsel.sum()))
            maxg.append(int(np.bincount(sel).max()))
        for i in range(args.warmup):
            ctx.forward(weights(i % args.layers, M), x, out[:M])
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # eager launches (host-side launch cost included)
        ev0.record(stream)
        for i in range(args.steps):
            ctx.forward(weights(i % args.layers, M), x, out[:M])
        ev1.record(stream)
        torch.cuda.synchronize()
        per_eager = ev0.elapsed_time(ev1) / args.steps
        per = per_eager
        if not args.eager:
            # the same K steps captured once into a HIP graph (as a decode loop would run them),
            # replayed once untimed and once timed
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(args.steps):
                    ctx.forward(weights(i % args.layers, M), x, out[:M])
            g.replay()
            torch.cuda.synchronize()
            ev0.record(stream)
            g.replay()
            ev1.record(stream)
            torch.cuda.synchronize()
            per = ev0.elapsed_time(ev1) / args.steps
            del g
        nbytes = sum(layer_bytes(touched[i % args.layers], M) for i in range(args.steps)) / args.steps
        nops = sum(layer_ops(ents[i % args.layers], M) for i in range(args.steps)) / args.steps
        # per-kernel durations: each kernel of the sequence alone, launched K times back to back
        # over the same layer rotation, between two events on the launch stream (the workspace
        # holds the last forward's routing and activations, so every launch does a real call's
        # work on cold weights); the K launches are captured into a HIP graph so that host launch
        # cost does not hide short kernels
        ctx.set_timing(True)  # the kernels this M launches
        ctx.forward(weights(0, M), x, out[:M])
        names = list(ctx.timing())
        ctx.set_timing(False)
        kern = {}
        for name in names:
            ctx.forward(weights(0, M), x, out[:M])
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(args.steps):
                    ctx.launch_kernel(name, weights(i % args.layers, M), x, out[:M])
            g.replay()
            torch.cuda.synchronize()
            ev0.record(stream)
            g.replay()
            ev1.record(stream)
            torch.cuda.synchronize()
            kern[name] = (ev0.elapsed_time(ev1), args.steps)
            del g
        results[M] = dict(
            tokens_per_s=M / (per * 1e-3), us_per_layer=per * 1e3, us_per_layer_eager=per_eager * 1e3,
            layer_GBps=nbytes / (per * 1e-3) / 1e9,
            hbm_frac=nbytes / (per * 1e-3) / 1e9 / HBM_PEAK_GBS, int8_TOPS=nops / (per * 1e-3) / 1e12,
            mfma_frac=nops / (per * 1e-3) / 1e12 / INT8_PEAK_TOPS, experts_touched=float(np.mean(touched)),
            layer_MB=nbytes / 1e6,
            kernels_us={k: round(v[0] / v[1] * 1e3, 2) for k, v in kern.items()},
            largest_group=float(np.mean(maxg)),
            routing=("Zipf(1.1) load: per-rank router bias fitted to Plackett-Luce top-10 inclusion "
                     "(trmoe/zipf_bias_table.json)" if M >= 512 else "router logits only (no bias)"),
            _kern=kern, _touched=touched, _ents=ents)
        log(f"M={M}: {per * 1e3:.1f} us/layer (eager {per_eager * 1e3:.1f}), {M / (per * 1e-3):.0f} tok/s, "
            f"{nbytes / (per * 1e-3) / 1e9:.0f} GB/s, kernels {results[M]['kernels_us']}")

    extras = {}
    todo = {v for v in args.extra.split(",") if v}
    if "c4" in todo:
        extras["C4 M=3072"] = bench_config4(args, layers, dev, stream, trmoe, torch, np)
    for key, fmt, nm in (("q80", trmoe.FMT_Q8_0, "Q8_0"), ("q51", trmoe.FMT_Q5_1, "Q5_1"),
                         ("q6k", trmoe.FMT_Q6_K, "Q6_K")):
        if key in todo:
            for Md, res in bench_down_format(args, layers, fmt, nm, dev, stream, trmoe, torch).items():
                extras[f"{nm} down M={Md}"] = res
    if "tq" in todo:
        for Mt, res in bench_tq(args, dev, stream, trmoe, torch, np).items():
            extras[f"TQ real shape M={Mt}"] = res
    if "hc" in todo:
        for Mh, res in bench_hc(args, dev, stream, trmoe, torch, np).items():
            extras[f"hc mix + TQ layer M={Mh}"] = res
    if "gemv" in todo:
        extras["trk_gemv dense projections"] = bench_gemv(args, dev, stream, trmoe, torch, np)
    if "stack" in todo:
        for Ms in (1, 512):
            extras[f"C5 stack M={Ms}"] = bench_stack(args, layers, ctx if Ms <= m_max else None, Ms, dev, stream,
                                                     trmoe, torch)

    prim = 1 if 1 in results else ms_list[0]
    r = results[prim]
    # roofline of the dominant kernel of the primary workload, and of every other M
    roofs = {M: roofline(M, res, np) for M, res in results.items()}
    roof = roofs[prim]
    for M, res in results.items():
        if M != prim:
            res["roofline"] = roofs[M]

    cpu = None
    if not args.no_cpu and prim == 1:
        cpu = cpu_baseline(layers[0], xs[1], args.cpu_seconds, trmoe.zipf_bias(1, E))

    line = {
        "metric": "MoE-layer tokens/s (decode M=1; M=4/8/16/512 in results)",
        "value": round(r["tokens_per_s"], 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["us_per_layer"] / 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"MoE layer M={prim}: H={H} E={E} F={F} top-{K} + shared expert, Q4_K gate/up/down, "
                               f"fp32 router; {args.layers}-layer rotation (config 5 stack) to defeat the MALL",
                   "hidden": H, "n_expert": E, "n_ff": F, "top_k": K, "M": prim, "layers": args.layers,
                   "parallelism": "single GPU"},
        "roofline": roof, "cpu_baseline": cpu,
        "results": {f"M={M}": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()
                               if not k.startswith("_")} for M, res in results.items()},
    }
    line["results"].update(extras)
    print(json.dumps(line), flush=True)
    if args.copy_cal:
        n = args.copy_cal << 18  # floats
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copies: 3 x {args.copy_cal} MiB")


def timed_graph(torch, stream, body, reps):
    """Capture body() once into a HIP graph, replay it once untimed, then `reps` times between
    events on the launch stream; returns ms per replay."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / reps


def bench_config4(args, layers, dev, stream, trmoe, torch, np):
    """Config 4: M=3072 tokens, gate/up Q4_K and down Q6_K, dynamic-k routing (smallest k whose
    cumulative router mass reaches 0.9, clamped to 1..10, MassBasis::Top), over the same layer
    rotation with Q6_K down projections."""
    M = 3072
    t0 = time.time()
    lw = [w.with_down(trmoe.FMT_Q6_K, 1, l, device=dev) for l, w in enumerate(layers)]
    for w in lw:
        w.moew.router_bias = None
    ctx = trmoe.Context(H, E, F, K, M)
    if args.stream_rows is not None:
        ctx.set_stream_rows(args.stream_rows)
    ctx.set_moe((1, K, 0.9, trmoe.BASIS_TOP))
    x = trmoe.gen_normal(1, (9 << 32) | M, M * H, 1.0, device=dev).view(M, H)
    out = torch.empty((M, H), dtype=torch.float32, device=dev)
    touched, ents = [], []
    for l in range(len(lw)):
        ctx.forward(lw[l], x, out)
        ng, n_ent = ctx.read(trmoe.WS_NGROUPS, 16, np.uint32)[:2]
        touched.append(int(ng))
        ents.append(int(n_ent))
    torch.cuda.synchronize()
    log(f"config 4: {len(lw)} layers with Q6_K down in {time.time() - t0:.1f}s; "
        f"mean k {np.mean(ents) / M:.2f}, touched {np.mean(touched):.0f}")
    steps = min(args.steps, 2 * len(lw))

    def body():
        for i in range(steps):
            ctx.forward(lw[i % len(lw)], x, out)

    per = timed_graph(torch, stream, body, 1) / steps
    dn = H * (F // 256 * 210)  # Q6_K down bytes per expert
    nbytes = float(np.mean(touched) + 1) * (2 * F * Q4K_ROW_H + dn) + E * H * 4 + H * 4 + M * H * 4 * 2
    nops = (float(np.mean(ents)) + M) * 3 * 2 * H * F
    # per-kernel times (each kernel alone over the rotation) and the dominant kernel's roofline
    ctx.set_timing(True)
    ctx.forward(lw[0], x, out)
    names = list(ctx.timing())
    ctx.set_timing(False)
    kern = {}
    for name in names:
        ctx.forward(lw[0], x, out)

        def kbody():
            for i in range(steps):
                ctx.launch_kernel(name, lw[i % len(lw)], x, out)

        kern[name] = timed_graph(torch, stream, kbody, 1) / steps
    ctx.close()
    del lw
    dom = max(kern, key=kern.get)
    nent, tch = float(np.mean(ents)), float(np.mean(touched)) + 1
    act = (nent + M) * (F + F // 16 * 12)
    alg = {"batch_gateup": tch * 2 * F * Q4K_ROW_H + M * (H + H // 32 * 12) + act,
           "batch_down": tch * dn + act + (nent + M) * H * 4}.get(dom)
    roof = None
    if alg:
        ach = alg / (kern[dom] * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom, M),
                "alg_bytes_per_launch": int(alg), "avg_launch_us": round(kern[dom] * 1e3, 2)}
    log(f"config 4: {per * 1e3:.1f} us/layer, kernels {({k: round(v * 1e3, 2) for k, v in kern.items()})}")
    return {"tokens_per_s": round(M / (per * 1e-3), 1), "us_per_layer": round(per * 1e3, 2),
            "layer_GBps": round(nbytes / (per * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (per * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "int8_TOPS": round(nops / (per * 1e-3) / 1e12, 3), "mean_k": round(float(np.mean(ents)) / M, 3),
            "experts_touched": round(float(np.mean(touched)), 1), "layers": len(layers), "steps": steps,
            "kernels_us": {k: round(v * 1e3, 2) for k, v in kern.items()}, "roofline": roof}


def bench_down_format(args, layers, fmt, name, dev, stream, trmoe, torch):
    """The layer with its down projections (routed and shared) regenerated in another GGUF format,
    at M=1 (no router bias) and M=512 (the Zipf bias), over the same layer rotation."""
    lw = [w.with_down(fmt, 1, l, device=dev) for l, w in enumerate(layers)]
    bias = torch.from_numpy(trmoe.zipf_bias(1, E)).to(dev)
    out_res = {}
    for M in (1, 512):
        for w in lw:
            w.moew.router_bias = bias.data_ptr() if M >= 64 else None
        ctx = trmoe.Context(H, E, F, K, M)
        if args.stream_rows is not None:
            ctx.set_stream_rows(args.stream_rows)
        x = trmoe.gen_normal(1, (9 << 32) | M, M * H, 1.0, device=dev).view(M, H)
        out = torch.empty((M, H), dtype=torch.float32, device=dev)
        ctx.forward(lw[0], x, out)
        steps = min(args.steps, 2 * len(lw))

        def body():
            for i in range(steps):
                ctx.forward(lw[i % len(lw)], x, out)

        per = timed_graph(torch, stream, body, 1) / steps
        ctx.close()
        out_res[M] = {"tokens_per_s": round(M / (per * 1e-3), 1), "us_per_layer": round(per * 1e3, 2),
                      "layers": len(lw), "steps": steps}
        log(f"{name} down M={M}: {per * 1e3:.1f} us/layer")
    del lw
    return out_res


def bench_tq(args, dev, stream, trmoe, torch, np):
    """The layer on the reference's own packed TQ experts at the real expert shape: H = 2560,
    F = 640, E = 512, top-10, gate/up TQ4_32 and down TQ5_16 (python/tests/test_blocks_real.py:
    23-26), over a rotation of args.tq_layers layers (synthetic packs generated on the GPU), at M = 1,
    M = 4 (each token as a decode) and M = 512 (Zipf-biased router)."""
    Ht, Et, Ft = 2560, 512, 640
    gf, df = trmoe.FMT_TQ4_32, trmoe.FMT_TQ5_16
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    t0 = time.time()
    lw = []
    for _ in range(args.tq_layers):
        lw.append(trmoe.LayerWeights.generate_tq(gen, Ht, Et, Ft, gf, df, device=dev))
    torch.cuda.synchronize()
    per_expert = 2 * trmoe.matrix_bytes(gf, Ft, Ht) + trmoe.matrix_bytes(df, Ht, Ft)
    log(f"TQ layers: {len(lw)} x {Et} experts ({len(lw) * Et * per_expert / 1e9:.1f} GB) in {time.time() - t0:.1f}s")
    bias = torch.from_numpy(trmoe.zipf_bias(1, Et)).to(dev)
    res = {}
    for M in (1, 4, 512):
        for w in lw:
            w.moew.router_bias = bias.data_ptr() if M >= 64 else None
        ctx = trmoe.Context(Ht, Et, Ft, K, M)
        x = torch.randn((M, Ht), device=dev, generator=gen)
        out = torch.empty((M, Ht), dtype=torch.float32, device=dev)
        touched = []
        for w in lw:
            ctx.forward(w, x, out)
            ids = ctx.read(trmoe.WS_IDS, M * 32 * 4, np.uint32).reshape(M, 32)
            nsel = ctx.read(trmoe.WS_NSEL, M * 4, np.uint32)
            touched.append(len(np.unique(np.concatenate([ids[t, :nsel[t]] for t in range(M)]))))
        steps = min(args.steps, 2 * len(lw))

        def body():
            for i in range(steps):
                ctx.forward(lw[i % len(lw)], x, out)

        per = timed_graph(torch, stream, body, 1) / steps
        ctx.set_timing(True)
        ctx.forward(lw[0], x, out)
        names = list(ctx.timing())
        ctx.set_timing(False)
        kern = {}
        for name in names:
            ctx.forward(lw[0], x, out)

            def kbody():
                for i in range(steps):
                    ctx.launch_kernel(name, lw[i % len(lw)], x, out)

            kern[name] = round(timed_graph(torch, stream, kbody, 1) / steps * 1e3, 2)
        ctx.close()
        nbytes = (float(np.mean(touched)) + 1) * per_expert + Et * Ht * 4 + M * Ht * 8
        res[M] = {"tokens_per_s": round(M / (per * 1e-3), 1), "us_per_layer": round(per * 1e3, 2),
                  "layer_GBps": round(nbytes / (per * 1e-3) / 1e9, 1),
                  "hbm_frac": round(nbytes / (per * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "experts_touched": round(float(np.mean(touched)), 1), "kernels_us": kern, "layers": len(lw),
                  "steps": steps}
        log(f"TQ real shape M={M}: {per * 1e3:.1f} us/layer, {M / (per * 1e-3):.0f} tok/s, kernels {kern}")
    del lw
    return res


def bench_hc(args, dev, stream, trmoe, torch, np):
    """8(f)1, the router input's producer: trk_moe_forward_hc (the hyper-connection mix part B,
    exec.rs:1196-1234 / exec_batch.rs:929-968, as the layer's input stage) on the real model's
    shapes: hc = 4 streams, low rank 320, H = 2560, then the TQ layer (E = 512, F = 640, TQ4_32 /
    TQ5_16), over a rotation of 8 layers (14 GB of experts), at M = 1 and M = 512.  The mix's up
    projection [hc H][lr] is TQ8_32.  Reports the layer with the mix, the layer alone on the first
    layer's mixed rows, and the hc_mix stage (at M >= 2 the lo quantisation and the mix kernel) with
    its roofline (the up matrix, xn, lo and the mixed rows)."""
    Ht, Et, Ft, hc, lr = 2560, 512, 640, 4, 320
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    ufmt = trmoe.FMT_TQ8_32
    lw, ups = [], []
    for _ in range(8):
        lw.append(trmoe.LayerWeights.generate_tq(gen, Ht, Et, Ft, device=dev))
        ups.append((trmoe.gen_tq_stack(gen, 1, hc * Ht, lr, ufmt, dev)[0], ufmt))
    ub = trmoe.matrix_bytes(ufmt, hc * Ht, lr)
    bias = torch.from_numpy(trmoe.zipf_bias(1, Et)).to(dev)
    res = {}
    for M in (1, 512):
        for w in lw:
            w.moew.router_bias = bias.data_ptr() if M >= 64 else None
        ctx = trmoe.Context(Ht, Et, Ft, K, M)
        xn = torch.randn((M, hc, Ht), device=dev, generator=gen)
        lo = torch.randn((M, lr), device=dev, generator=gen)
        out = torch.empty((M, Ht), dtype=torch.float32, device=dev)
        steps = min(args.steps, 2 * len(lw))
        ctx.forward_hc(lw[0], ups[0], hc, lr, xn, lo, out)
        # the layer alone runs on the mixed rows themselves, so both legs route the same tokens
        torch.cuda.synchronize()
        xm = torch.from_numpy(ctx.read(trmoe.WS_MIXED, M * Ht * 4, np.float32).reshape(M, Ht).copy()).to(dev)

        def body_hc():
            for i in range(steps):
                ctx.forward_hc(lw[i % len(lw)], ups[i % len(ups)], hc, lr, xn, lo, out)

        def body_plain():
            for i in range(steps):
                ctx.forward(lw[i % len(lw)], xm, out)

        per_hc = timed_graph(torch, stream, body_hc, 1) / steps
        per = timed_graph(torch, stream, body_plain, 1) / steps
        ctx.set_timing(True)
        for i in range(steps):
            ctx.forward_hc(lw[i % len(lw)], ups[i % len(ups)], hc, lr, xn, lo, out)
        mix_ms, n = ctx.timing()["hc_mix"]
        ctx.set_timing(False)
        ctx.close()
        mix_us = mix_ms / n * 1e3
        nbytes = ub + M * hc * Ht * 4 + M * lr * 4 + M * Ht * 4
        ach = nbytes / (mix_us * 1e-6) / 1e9
        res[M] = {"tokens_per_s": round(M / (per_hc * 1e-3), 1), "us_per_layer_with_mix": round(per_hc * 1e3, 2),
                  "us_per_layer_without": round(per * 1e3, 2), "hc_mix_us": round(mix_us, 2),
                  "roofline": {"bound": "hbm", "kernel": "hc_mix", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                               "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                               "alg_bytes_per_launch": int(nbytes), "avg_launch_us": round(mix_us, 2),
                               "timing": "per-launch events around each hc_mix launch (eager)"},
                  "layers": len(lw), "steps": steps, "hc": hc, "lr": lr, "up_fmt": "TQ8_32"}
        log(f"hc mix M={M}: layer {per_hc * 1e3:.1f} us with the mix, {per * 1e3:.1f} without; "
            f"hc_mix {mix_us:.2f} us ({ach:.0f} GB/s)")
    del lw, ups
    return res


def bench_gemv(args, dev, stream, trmoe, torch, np):
    """8(f)4: trk_gemv (gemv_tq_rows, gemv.rs:25-40) on the real model's dense projections at
    decode (one token, two-level activations as TR_HIPREC quantises them), the matrices as a pack
    holds them for one tile: the LM head (exec.rs:873, 1079) [248320][2560], attention q with its gate
    (exec.rs:1376) [12288][2560], the GDN qkv (exec.rs:1252) [10240][2560], the hyper-connection low-
    rank down (exec.rs:1181) [320][10240] and up (exec.rs:1214) [10240][320].  Each is timed over a
    rotation of copies totalling at least 600 MB (the 256 MB MALL cannot hold it), with a roofline
    (the matrix, the activations and the output per call)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(13)
    shapes = [("lm_head", 248320, 2560, trmoe.FMT_TQ8_32), ("attn_q", 12288, 2560, trmoe.FMT_TQ5_32),
              ("gdn_qkv", 10240, 2560, trmoe.FMT_TQ5_32), ("hc_down", 320, 10240, trmoe.FMT_TQ8_32),
              ("hc_up", 10240, 320, trmoe.FMT_TQ8_32)]
    res = {}
    for name, rows, k, fmt in shapes:
        mb = trmoe.matrix_bytes(fmt, rows, k)
        copies = max(1, min(256, -(-600_000_000 // mb)))
        wt = trmoe.gen_tq_stack(gen, copies, rows, k, fmt, dev)
        x = torch.randn(k, device=dev, generator=gen)
        q, s, su = trmoe.quantize(x, 32, pair=True)
        y = torch.empty((1, (rows + 15) // 16 * 16), dtype=torch.float32, device=dev)
        steps = max(copies, min(args.steps, 64))
        trmoe.gemv(wt, rows, k, fmt, 0, copies, 32, q, s, su, pair=True, y=y)

        def body():
            for i in range(steps):
                trmoe.gemv(wt, rows, k, fmt, i % copies, copies, 32, q, s, su, pair=True, y=y)

        us = timed_graph(torch, stream, body, 1) / steps * 1e3
        nbytes = mb + 2 * k + 2 * (k // 32) * 8 + rows * 4
        ach = nbytes / (us * 1e-6) / 1e9
        res[name] = {"rows": rows, "k": k, "fmt": f"TQ{fmt >> 8}_{fmt & 0xff}", "MB": round(mb / 1e6, 2),
                     "us": round(us, 2), "GBps": round(ach, 1),
                     "roofline": {"bound": "hbm", "kernel": "gemv_rows_kernel", "achieved": round(ach, 1),
                                  "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                                  "traffic": None, "alg_bytes_per_launch": int(nbytes), "avg_launch_us": round(us, 2)},
                     "copies": copies, "steps": steps}
        log(f"gemv {name} [{rows}][{k}] {res[name]['fmt']}: {us:.2f} us, {ach:.0f} GB/s")
        del wt
    return res


def bench_stack(args, layers, ctx, M, dev, stream, trmoe, torch):
    """Config 5: the whole stack, h <- h + MoE(RMSNorm(h; eps 1e-6, w ~ U(0.9, 1.1))) for each of
    the layers in turn, on seeded N(0, 1) rows, timed end to end (one replay = one pass)."""
    if ctx is None:
        ctx = trmoe.Context(H, E, F, K, M)
        if args.stream_rows is not None:
            ctx.set_stream_rows(args.stream_rows)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    rms = [torch.rand(H, generator=gen, device=dev) * 0.2 + 0.9 for _ in layers]
    for w in layers:
        w.moew.router_bias = None
    h = trmoe.gen_normal(1, (11 << 32) | M, M * H, 1.0, device=dev).view(M, H)

    def body():
        for l, w in enumerate(layers):
            ctx.residual(w, rms[l], 1e-6, h)

    reps = 20 if M == 1 else 3
    per = timed_graph(torch, stream, body, reps)
    ok = bool(torch.isfinite(h).all())
    log(f"config 5 stack M={M}: {per:.3f} ms per pass of {len(layers)} layers")
    return {"tokens_per_s": round(M / (per * 1e-3), 1), "ms_per_pass": round(per, 4),
            "us_per_layer": round(per * 1e3 / len(layers), 2), "layers": len(layers), "passes": reps,
            "finite": ok}


def roofline(M, res, np):
    """The roofline object of the dominant kernel of one M's layer: algorithmic bytes per launch
    (touched experts' weights, each byte once, plus the activations the kernel moves) over its
    average isolated launch time, against the 8 TB/s HBM peak; traffic from the counter passes."""
    kern = res["_kern"]
    dom = max(kern, key=lambda k: kern[k][0])
    avg_ms = kern[dom][0] / kern[dom][1]
    tavg = float(np.mean(res["_touched"]))
    nent = float(np.mean(res["_ents"]))
    gu_bytes = (tavg + 1) * 2 * F * Q4K_ROW_H
    dn_bytes = (tavg + 1) * H * Q4K_ROW_F
    xq = M * (H + H // 32 * 12)                # int8 x rows with their scale, sum and u
    act = (nent + M) * (F + F // 16 * 12)      # int8 SwiGLU rows with their scale, sum and u
    alg = {"decode_layer": gu_bytes + dn_bytes + E * H * 4 + H * 4 + H * 4 * 2,
           "decode_gateup": gu_bytes + 2 * 2 * H + 2 * (H // 32) * 8 + 33 * 2 * (F + F // 16 * 8),
           "decode_down": dn_bytes + (tavg + 1) * 2 * (F + F // 16 * 8) + H * 4,
           "batch_gateup": gu_bytes + xq + act, "batch_down": dn_bytes + act + (nent + M) * H * 4,
           "stream_gateup": gu_bytes + xq + act, "stream_down": dn_bytes + act + (nent + M) * H * 4,
           "router_logits": E * H * 4 + M * H * 4 + M * E * 4}.get(dom)
    if not alg:
        return None
    ach = alg / (avg_ms * 1e-3) / 1e9
    return {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom, M),
            "alg_bytes_per_launch": int(alg), "avg_launch_us": round(avg_ms * 1e3, 2)}


def measured_traffic(kernel, m):
    """HBM bytes per launch of `kernel` at M = m from the committed rocprofv3 counter passes
    (profiles/traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a copy kernel of known
    size), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return t[f"{kernel}@M={m}"]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def host_info(cpus):
    """CPU model and the NUMA nodes of the CPUs the baseline's threads are pinned to."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nodes = set()
    for c in cpus:
        try:
            nodes.update(int(d[4:]) for d in os.listdir(f"/sys/devices/system/cpu/cpu{c}") if d.startswith("node"))
        except (OSError, ValueError):
            pass
    return model, sorted(nodes)


def cpu_baseline(w, x_dev, seconds, bias=None):
    """The reference's CPU MoE layer timed on this host: moe_block (decode, M = 1) and moe_batch
    (M = 512) restated with AVX-512 VNNI over a pool of pinned threads (one tile of at most 16
    cores, the reference's T = 1 layout; oracle/cpu_moe.c), on layer 0's weights.  Each leg runs for
    about `seconds`.  A host without AVX-512 VNNI times the scalar C oracle on one core instead."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    t = w.tensors
    gate, up, down = t["gate"].cpu().numpy(), t["up"].cpu().numpy(), t["down"].cpu().numpy()
    orc = O.OracleLayer(H, E, F, t["router"].cpu().numpy().reshape(E, H), t["shexp_gate"].cpu().numpy(),
                        gate, up, down, t["sh_gate"].cpu().numpy(), t["sh_up"].cpu().numpy(),
                        t["sh_down"].cpu().numpy())
    x0 = x_dev.cpu().numpy()[0]
    rng = np.random.default_rng(0)
    xs = [x0] + [(x0 * rng.choice([-1.0, 1.0], H)).astype(np.float32) for _ in range(255)]
    vnni = O.cpu_have_vnni()
    if not vnni:
        for xx in xs[:64]:  # weight re-layout is offline in the reference: do it before timing
            orc.ensure(O.route_topk(orc.logits(xx, True)[0], K)[0])
        n, spent = 0, 0.0
        while n < 64 and (spent < seconds or n < 2):
            ts = time.perf_counter()
            orc.moe_block(xs[n], k=K, hiprec=True)
            spent += time.perf_counter() - ts
            n += 1
        return {"value": round(n / spent, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"{n} decode tokens (M=1) of layer 0 through the scalar C oracle (this host has no "
                          f"AVX-512 VNNI)", "seconds": round(spent, 2)}

    # weight re-layout (GGUF -> TQ) is offline in the reference: every expert before timing
    t0 = time.perf_counter()
    orc.ensure(range(E))
    conv = time.perf_counter() - t0
    cm = O.CpuMoe(0)
    try:
        amx = bool(cm.L.cpu_amx_available())
        model, nodes = host_info(cm.cpus)
        # decode: M = 1 tokens one after another (moe_block, exec.rs:1540-1623)
        for xx in xs[:4]:
            cm.block(orc, xx, K)
        n, spent = 0, 0.0
        while spent < seconds / 2 or n < 8:
            ts = time.perf_counter()
            cm.block(orc, xs[n % len(xs)], K)
            spent += time.perf_counter() - ts
            n += 1
        # batch: M = 512 with the Zipf router bias the GPU leg uses (moe_batch, exec_batch.rs:1404-1580)
        orc.router_bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        xb = np.ascontiguousarray(rng.standard_normal((512, H)), np.float32)
        cm.batch(orc, xb, K)
        nb, sb = 0, 0.0
        while sb < seconds / 2 or nb < 1:
            ts = time.perf_counter()
            cm.batch(orc, xb, K)
            sb += time.perf_counter() - ts
            nb += 1
        orc.router_bias = None
    finally:
        threads, cpus = cm.threads, cm.cpus
        cm.close()
    return {"value": round(n / spent, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "m512_tokens_per_s": round(nb * 512 / sb, 1),
            "sample": f"{n} decode tokens (M=1, moe_block, {len(xs)} distinct inputs in turn) and {nb} batch(es) of M=512 (moe_batch, Zipf-biased "
                      f"router) of layer 0 through the AVX-512 VNNI restatement of the reference's CPU path "
                      f"(oracle/cpu_moe.c) on one tile of {threads} pinned threads; GGUF->TQ re-layout of all "
                      f"{E} experts done beforehand ({conv:.1f} s), as the reference packs offline",
            "host": {"cpu": model, "cpus": cpus, "numa_nodes": nodes, "avx512_vnni": True,
                     "amx": "available, unused: the reference's routed experts run VNNI" if amx else
                            "unavailable -> VNNI timed"},
            "seconds": round(spent + sb, 2)}


if __name__ == "__main__":
    main()
