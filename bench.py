#!/usr/bin/env python3
"""Benchmark of the MI355X MoE block (BASELINE.json metric).

Headline (`value`): MoE-layer decode tokens/s at B=1 on the Qwen3.6-35B-A3B-shaped layer
(config c1: H2048, E256, top-8, I512, shared 512, 4-bit g64).  A step pushes one fresh
token through a chain of `--layers` distinct seeded layers (40 x 453 MB of expert pages,
so the step's ~640 MB of selected pages come from HBM, not the 256 MB Infinity Cache);
each step is one captured HIP graph.  value = layers * steps / timed seconds.

Also reported: prefill of 2048 tokens (config c2) with per-stage times and the roofline of its
two GEMM launches (prefill_roofline: FLOPs per launch over the attributed stage time, against
the dense bf16 MFMA peak), the roofline of the dominant decode kernel (its average duration
from start/stop events attached to its own dispatches over K x L eager calls; HBM traffic per
launch from the rocprofv3 counter summaries profiles/decode_traffic.json and
profiles/prefill_c2_t2048_traffic.json when present), and the CPU oracle (C restatement of the
reference op graph): decode and a c2 prefill sample on every usable host core and on one,
medians of 5 runs.
--copy-check first runs a plain 1 GiB device-to-device copy three times: the reference
dispatch that scales the FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run.
--prefill-only runs the c2 prefill alone (the workload of the prefill counter profiles);
--counter-summary DIR... prints a per-kernel table of rocprofv3 --pmc output and exits.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
# attributed stage -> decode kernel that carries it (the other stages run inside these)
DECODE_KERNELS = {"router": "decode_router_kernel", "gate_up": "decode_gate_up_kernel",
                  "down": "decode_down_kernel"}
BF16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=40)
    p.add_argument("--prefill-iters", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-extra", action="store_true",
                   help="skip the side measurements of configs c3 and c4")
    p.add_argument("--verification-only", action="store_true",
                   help="only the MTP verification QMV measurement (one JSON line of its own)")
    p.add_argument("--cpu-seconds", type=float, default=20.0,
                   help="budget of the CPU baseline's decode runs (the prefill samples come on top)")
    p.add_argument("--copy-check", action="store_true",
                   help="run a 1 GiB streaming copy first (counter calibration)")
    p.add_argument("--prefill-only", action="store_true",
                   help="only the c2 prefill (one JSON line of its own): the workload of the prefill "
                        "counter profiles")
    p.add_argument("--counter-summary", nargs="+", metavar="DIR",
                   help="summarise rocprofv3 --pmc output directories per kernel (markdown) and exit")
    return p.parse_args()


def main():
    args = parse()
    if args.counter_summary:
        print(counter_summary(args.counter_summary))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the MoE block's multi-GPU "
                          "sharding (expert parallelism over RCCL) is designed, not built; "
                          "run with --gpus 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    from astronomical_amd import configs as CF
    from astronomical_amd import device_synthetic as DS
    from astronomical_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.verification_only:
        print(json.dumps(verification_qmv(CF, DS, ops, torch)))
        return
    if args.copy_check:
        # a plain streaming kernel of known traffic: reads 1 GiB, writes 1 GiB
        a = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            torch.mul(a, 1.0, out=b)
        torch.cuda.synchronize()
        del a, b
        log("copy check: 3 x (1 GiB read + 1 GiB write) elementwise kernel")
    cfg = CF.C1
    nL, K, W = args.layers, args.steps, args.warmup
    if args.prefill_only:
        blk = ops.MoeBlock(DS.make_layer_device(cfg, layer=0))
        print(json.dumps(prefill_c2(CF, DS, torch, blk, args.prefill_iters)))
        return

    # ---------------------------------------------------------------- decode chain
    layers = [DS.make_layer_device(cfg, layer=l) for l in range(nL)]
    log(f"generated {nL} layers of {cfg.name}")
    blocks = [ops.MoeBlock(L) for L in layers]
    ws = blocks[0].workspace(2048)
    for b in blocks:
        b._ws = ws
    toks = DS.make_tokens_device(cfg, (K + W) * nL, step=1).reshape(K + W, nL, 1, cfg.hidden)
    outs = torch.empty(nL, 1, cfg.hidden, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    def run_step(s):
        for l in range(nL):
            blocks[l].forward(toks[s, l], out=outs[l], workspace=ws)

    # eager reference of step 0, then capture one graph per step
    run_step(0)
    torch.cuda.synchronize()
    eager0 = outs.clone()
    graphs = []
    for s in range(K + W):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run_step(s)
        graphs.append(g)
    # replays must reproduce eager results, with eager work in between
    for _ in range(3):
        outs.zero_()
        graphs[0].replay()
        torch.cuda.synchronize()
        assert torch.equal(outs, eager0), "graph replay differs from eager execution"
        run_step(1)
        torch.cuda.synchronize()

    log(f"captured {K + W} step graphs; replay == eager")
    for s in range(W):
        graphs[s].replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(K):
        graphs[W + i].replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(K)]
    total_ms = ev[0].elapsed_time(ev[K])
    ms_per_step = total_ms / K
    ms_per_layer = ms_per_step / nL
    decode_tps = 1000.0 / ms_per_layer  # B = 1 token per layer step
    page = cfg.page_bytes
    credited = (cfg.top_k + 1) * page  # U = 8 distinct routed experts + the shared expert
    layer_gbs = credited / (ms_per_layer * 1e-3) / 1e9

    log(f"decode: {ms_per_layer * 1000:.2f} us/layer")
    # per-kernel device times of the same decode workload: eager calls of the attributed
    # entry point, whose decode kernels carry start/stop events on their own dispatches
    # (hipExtLaunchKernelGGL) on the stream they run on
    stage_acc = {}
    for s in range(W, W + K):
        for l in range(nL):
            _, st = blocks[l].forward_attributed(toks[s, l], out=outs[l], workspace=ws)
            for kname, v in st.items():
                stage_acc.setdefault(kname, []).append(v)
    stage_ms = {kname: statistics.mean(v) for kname, v in stage_acc.items()}
    kernel_ms = {DECODE_KERNELS[s_]: stage_ms[s_] for s_ in DECODE_KERNELS}
    # algorithmic bytes of one launch of each decode kernel at B=1 (weights read once each)
    H, I, Is, E, kk = cfg.hidden, cfg.intermediate, cfg.shared_intermediate, cfg.experts, cfg.top_k
    per_elem = cfg.bits / 8 + 4 / cfg.group_size  # codes + bf16 scale and bias per group
    kernel_bytes = {
        "decode_router_kernel": E * H * 2,
        "decode_gate_up_kernel": (kk * 2 * I * H + 2 * Is * H + H) * per_elem,
        "decode_down_kernel": (kk * H * I + H * Is) * per_elem,
    }
    dom = max(kernel_ms, key=lambda k_: kernel_ms[k_])
    dom_bytes = kernel_bytes[dom]
    dom_gbs = dom_bytes / (kernel_ms[dom] * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f).get(dom)
        if tr:
            traffic = int(tr["fetch_bytes"] + tr["write_bytes"])

    # ---------------------------------------------------------------- prefill 2048 (c2)
    pre = prefill_c2(CF, DS, torch, blocks[0], args.prefill_iters)
    log(f"prefill: {pre['prefill']['ms'] * 1000:.1f} us")

    # ---------------------------------------------------------------- side measurements
    extra = None
    if not args.no_extra:
        extra = decoder_step(CF, DS, ops, torch, blocks, K, W)
        extra["c1_decode_batched"] = batched_decode(CF, DS, ops, torch, blocks, K, W)
        extra["c1_decode_affine_router"] = affine_router_decode(CF, DS, ops, torch, layers, K, W)
        extra["c1_decode_paged"] = paged_decode(CF, ops, torch, layers, K, W)
        extra.update(other_configs(CF, DS, ops, torch, K, W, layers[0]))
        extra["verification_lm_head"] = verification_qmv(CF, DS, ops, torch)

    # ---------------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(layers[0], toks, cfg, DS.make_tokens_device(CF.C2, 64, step=2), args.cpu_seconds)

    result = {
        "metric": "MoE-layer tokens/s (decode B=1, prefill 2048) + % HBM/MFMA roofline, 1xMI355X",
        "value": round(decode_tps, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"c1 decode B=1: Qwen3.6-35B-A3B-shaped MoE layer (H2048 E256 top-8 I512 + shared 512, "
                        f"4-bit g64), one token per step through a chain of {nL} distinct seeded layers, "
                        f"one hipGraph per step",
            "layers_per_step": nL,
            "ms_per_layer": round(ms_per_layer, 5),
            "step_ms_median": round(statistics.median(step_ms), 4),
            "wall_s_timed": round(wall, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{dom} (decode B=1, c1)",
            "achieved": round(dom_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(dom_bytes),
            "avg_launch_us": round(kernel_ms[dom] * 1000, 2),
        },
        "layer_roofline": {
            "credited_bytes_per_layer": int(credited),
            "achieved_GBps": round(layer_gbs, 1),
            "frac_of_hbm_peak": round(layer_gbs / HBM_PEAK_GBS, 4),
        },
        "decode_kernel_us": {k_: round(v * 1000, 2) for k_, v in kernel_ms.items()},
        "decode_kernel_GBps": {k_: round(kernel_bytes[k_] / (v * 1e-3) / 1e9, 1) for k_, v in kernel_ms.items()},
        "prefill": pre["prefill"],
        "prefill_roofline": pre["prefill_roofline"],
        "other_configs": extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))


def prefill_c2(CF, DS, torch, blk, iters):
    """c2: 2048 tokens through one c1 layer (the sorted path).  Whole-block time from events
    around `iters` forwards; per-stage device times (median of 5) from the attributed entry
    point, whose gate/up and down stages are one GEMM launch each.  The roofline of those two
    launches: FLOPs of the routed and shared projections over the launch's duration, against
    the dense bf16 MFMA peak; HBM traffic per launch from the counter summary
    profiles/prefill_c2_t2048_traffic.json when present."""
    cfg, T = CF.C1, 2048
    xp = DS.make_tokens_device(CF.C2, T)
    yp = torch.empty_like(xp)
    wsp = blk.workspace(T)
    for _ in range(3):
        blk.forward(xp, out=yp, workspace=wsp)
    torch.cuda.synchronize()
    pe0, pe1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    pe0.record()
    for _ in range(iters):
        blk.forward(xp, out=yp, workspace=wsp)
    pe1.record()
    torch.cuda.synchronize()
    ms = pe0.elapsed_time(pe1) / iters
    flops = cfg.flops_per_token() * T
    pst = {}
    for _ in range(5):
        _, st = blk.forward_attributed(xp, out=yp, workspace=wsp)
        for kname, v in st.items():
            pst.setdefault(kname, []).append(v)
    stage_ms = {kname: statistics.median(v) for kname, v in pst.items()}
    H, I, Is, A = cfg.hidden, cfg.intermediate, cfg.shared_intermediate, T * cfg.top_k
    gemm_flops = {"gate_up": 2 * A * 2 * I * H + 2 * T * 2 * Is * H, "down": 2 * A * H * I + 2 * T * H * Is}
    names = {"gate_up": "xq_gemm_kernel<SwiGLU> (c2 routed + shared gate/up)",
             "down": "xq_gemm_kernel<plain> (c2 routed + shared down)"}
    traffic = {}
    tpath = os.path.join(ROOT, "profiles", "prefill_c2_t2048_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f)

    def entry(stage):
        us = stage_ms[stage] * 1000
        tf = gemm_flops[stage] / (us * 1e-6) / 1e12
        t = traffic.get(stage)
        return {"bound": "mfma", "kernel": names[stage], "achieved": round(tf, 2), "peak": BF16_DENSE_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tf / BF16_DENSE_PEAK_TFLOPS, 4),
                "traffic": int(t["fetch_bytes"] + t["write_bytes"]) if t else None,
                "flops_per_launch": int(gemm_flops[stage]), "avg_launch_us": round(us, 2)}
    dom = max(gemm_flops, key=lambda k_: stage_ms[k_])
    other = "down" if dom == "gate_up" else "gate_up"
    roof = entry(dom)
    roof["next"] = entry(other)
    return {"prefill": {
        "workload": "c2: c1 shapes, 2048 tokens, sorted path",
        "ms": round(ms, 4),
        "tokens_per_s": round(T / (ms * 1e-3), 1),
        "achieved_TFLOPs": round(flops / (ms * 1e-3) / 1e12, 2),
        "frac_of_bf16_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_DENSE_PEAK_TFLOPS, 4),
        "stage_us": {k_: round(v * 1000, 2) for k_, v in stage_ms.items()},
    }, "prefill_roofline": roof}


def counter_summary(dirs):
    """Per-kernel averages of rocprofv3 --pmc output (the *_counter_collection.csv files under
    each directory), as a markdown table: one row per kernel, one column per counter, values
    per dispatch.  Kernel names are cut at their argument list."""
    import csv
    import glob
    agg, disp = {}, {}
    for d in dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for r in csv.DictReader(f):
                    k = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
                    agg.setdefault(k, {}).setdefault(r["Counter_Name"], 0.0)
                    agg[k][r["Counter_Name"]] += float(r["Counter_Value"])
                    disp.setdefault(k, {}).setdefault(r["Counter_Name"], set()).add((path, r["Dispatch_Id"]))
    counters = sorted({c for k in agg for c in agg[k]})
    lines = ["| kernel | dispatches | " + " | ".join(counters) + " |", "|---|---|" + "---|" * len(counters)]
    for k in sorted(agg, key=lambda k_: -sum(agg[k_].values())):
        n = max(len(v) for v in disp[k].values())
        row = [f"{agg[k][c] / len(disp[k][c]):.6g}" if c in agg[k] else "" for c in counters]
        lines.append(f"| {k} | {n} | " + " | ".join(row) + " |")
    return "\n".join(lines)


def other_configs(CF, DS, ops, torch, K, W, layer_c1):
    """c3 (4096-token prefill with Zipf-skewed routing), c4 (48 stacked 8-bit layers: decode
    B=1 through a graph of all 48, and 512-token prefill per layer), timed with events, and
    the expert page loader (a c1 decode page from a safetensors checkpoint into HBM)."""
    out = {"expert_page_load": page_load(CF, torch, layer_c1)}

    def prefill_entry(cfg, T, us):
        tf = cfg.flops_per_token() * T / (us * 1e-6) / 1e12
        return {"tokens": T, "us_per_layer": round(us, 1), "tokens_per_s": round(T / (us * 1e-6), 1),
                "achieved_TFLOPs": round(tf, 2), "frac_of_bf16_peak": round(tf / BF16_DENSE_PEAK_TFLOPS, 4)}

    def time_ms(fn, iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    # c3: skewed routing (router bias 2 ln Zipf(1.1) rank weights), 4096 tokens
    c3 = CF.C3
    L3 = DS.make_layer_device(c3, layer=0)
    b3 = ops.MoeBlock(L3)
    x3 = DS.make_tokens_device(c3, 4096)
    y3 = torch.empty_like(x3)
    ws3 = b3.workspace(4096)
    ms = time_ms(lambda: b3.forward(x3, out=y3, workspace=ws3), 10)
    out["c3_prefill"] = dict(workload="c3: c1 shapes, 4096 tokens, Zipf-skewed routing", **prefill_entry(c3, 4096, ms * 1000))
    del L3, b3, x3, y3, ws3

    # c4: 48 stacked 8-bit layers
    c4 = CF.C4
    nL4 = c4.layers
    L4 = [DS.make_layer_device(c4, layer=l) for l in range(nL4)]
    b4 = [ops.MoeBlock(L) for L in L4]
    ws4 = b4[0].workspace(512)
    t4 = DS.make_tokens_device(c4, nL4, step=1).reshape(nL4, 1, c4.hidden)
    o4 = torch.empty_like(t4)

    def decode_pass():
        for l in range(nL4):
            b4[l].forward(t4[l], out=o4[l], workspace=ws4)
    decode_pass()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        decode_pass()
    for _ in range(W):
        g.replay()
    ms = time_ms(g.replay, K)
    us_layer = ms * 1000 / nL4
    credited = c4.top_k * c4.page_bytes  # 8 distinct routed expert pages, no shared expert
    gbs = credited / (us_layer * 1e-6) / 1e9
    out["c4_decode"] = {"workload": f"c4 decode B=1 through a graph of {nL4} distinct 8-bit layers",
                        "us_per_layer": round(us_layer, 2), "tokens_per_s_48_layers": round(1e6 / (us_layer * nL4), 1),
                        "credited_bytes_per_layer": int(credited), "achieved_GBps": round(gbs, 1),
                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    xp = DS.make_tokens_device(c4, 512)
    yp = torch.empty_like(xp)

    def prefill_pass():
        for l in range(nL4):
            b4[l].forward(xp, out=yp, workspace=ws4)
    ms = time_ms(prefill_pass, 3)
    us4 = ms * 1000 / nL4
    # at ~32 rows per expert this shape is bound by its weight bytes: every expert page (gate,
    # up, down codes + scales + biases) is read once per layer, plus the activations
    wbytes = c4.experts * c4.page_bytes + 512 * c4.hidden * 2 * 2
    gbs4 = wbytes / (us4 * 1e-6) / 1e9
    out["c4_prefill"] = dict(workload=f"c4: 512 tokens through each of {nL4} 8-bit layers",
                             **prefill_entry(c4, 512, us4), weight_bytes_per_layer=int(wbytes),
                             achieved_GBps=round(gbs4, 1), frac_of_hbm_peak=round(gbs4 / HBM_PEAK_GBS, 4))
    del L4, b4, ws4
    torch.cuda.empty_cache()
    log(f"other configs: {json.dumps(out)}")
    return out


def verification_qmv(CF, DS, ops, torch, reps=20, vocab=248_320):
    """The multi-token QMV of MTP target-verification windows on the largest linear that runs
    through it: the c1 model's logits head (hidden 2048 -> vocabulary 248,320, the Qwen3.5-MoE
    config of the reference's tests), 4-bit and 5-bit g64, for windows of 1..16 tokens.  A
    hipGraph of `reps` launches per point, timed with events; bytes = codes + scales + biases
    + activations + outputs (one pass over the weights per launch)."""
    H = CF.C1.hidden
    out = {"workload": f"MTP verification window (batch 1, T tokens) through the logits head "
                       f"{H} -> {vocab}, bf16 activations, affine g64 codes; one launch per window"}
    for bits in (4, 5):
        cfg = CF.C1.with_(bits=bits)
        w = DS.affine(cfg, cfg.seed, f"lm_head_{bits}", 1, vocab, H)
        codes, sc, bi = w.w[0], w.scales[0], w.biases[0]
        res = {}
        for T in (1, 2, 4, 8, 16):
            x = DS.normal_bf16(cfg.seed, f"verify_x_{T}", (1, T, H), 1.0)

            def fn():
                ops.qwen3_5_target_verification_quantized_linear(x, codes, sc, bi, cfg.group_size, bits)
            fn()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(reps):
                    fn()
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1000 / reps
            nbytes = vocab * H * bits // 8 + vocab * (H // cfg.group_size) * 4 + T * H * 2 + T * vocab * 2
            gbs = nbytes / (us * 1e-6) / 1e9
            res[f"T{T}"] = {"us": round(us, 2), "bytes": int(nbytes), "GBps": round(gbs, 1),
                            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
            del g
        out[f"{bits}bit"] = res
        del w, codes, sc, bi
        torch.cuda.empty_cache()
    # the MoE block over a verification window (every row bit-equal to its one-token block):
    # a hipGraph of the window through 40 distinct c1 layers, per-layer time
    nL = 40
    layers = [DS.make_layer_device(CF.C1, layer=l) for l in range(nL)]
    blocks = [ops.MoeBlock(L) for L in layers]
    blk_res = {}
    for T in (2, 4, 8):
        xs = DS.make_tokens_device(CF.C1, nL * T, step=7).reshape(nL, T, H)
        ys = torch.empty_like(xs)
        wsz = blocks[0].verification_workspace_bytes(T)
        ws = torch.empty(wsz, dtype=torch.uint8, device="cuda")

        def window_pass():
            for l in range(nL):
                blocks[l].target_verification_forward(xs[l], out=ys[l], workspace=ws)
        window_pass()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            window_pass()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us_layer = e0.elapsed_time(e1) * 1000 / (5 * nL)
        blk_res[f"T{T}"] = {"us_per_layer": round(us_layer, 2), "tokens_per_s": round(T / (us_layer * 1e-6), 1)}
        del g, xs, ys, ws
    out["block_window"] = {"workload": f"c1 MoE block in verification mode (rows unsorted, token-local), "
                                       f"a window of T tokens through a graph of {nL} distinct layers",
                           **blk_res}
    del layers, blocks
    torch.cuda.empty_cache()
    log(f"verification qmv: {json.dumps(out)}")
    return out


def batched_decode(CF, DS, ops, torch, blocks, K, W, sizes=(2, 4, 8)):
    """c1 decode at B = 2, 4, 8 tokens per step (production mode: the sorted combine at 64
    assignments) through a graph of all the layers, as the B = 1 headline.  Credited bytes per
    layer = (distinct routed experts of the step + the shared expert) x page bytes, the
    distinct experts counted from each layer's routing of the step's tokens."""
    import numpy as np
    cfg = CF.C1
    H, nL, dev = cfg.hidden, len(blocks), torch.device("cuda")
    out = {"workload": f"c1 decode, B tokens per step through a graph of {nL} distinct layers"}
    for B in sizes:
        x = DS.make_tokens_device(cfg, nL * B, step=11).reshape(nL, B, H)
        y = torch.empty_like(x)
        ws = torch.empty(blocks[0].workspace_bytes(B), dtype=torch.uint8, device=dev)
        distinct = []
        for l in range(nL):
            blocks[l].forward(x[l], out=y[l], workspace=ws)
            distinct.append(len(np.unique(blocks[l].trace(B, workspace=ws)["indices"])))

        def step():
            for l in range(nL):
                blocks[l].forward(x[l], out=y[l], workspace=ws)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        for _ in range(W):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(K):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / K / nL * 1000
        u = float(np.mean(distinct))
        credited = (u + 1) * cfg.page_bytes
        gbs = credited / (us * 1e-6) / 1e9
        out[f"B{B}"] = {"us_per_layer": round(us, 2), "tokens_per_s": round(B / (us * 1e-6), 1),
                        "distinct_experts": round(u, 2), "credited_bytes_per_layer": int(credited),
                        "achieved_GBps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        del g, x, y, ws
    log(f"batched decode: {json.dumps(out)}")
    return out


def paged_decode(CF, ops, torch, layers, K, W):
    """c1 decode B=1 with every layer's routed arrays as a compact page (paged_execution.rs:
    98-139): the page holds all of the layer's experts in a seeded permuted slot order and the
    block gets its slot map, so the decode kernels read each selected expert at its slot and
    sort the assignments by slot."""
    import copy
    cfg = CF.C1
    H, nL, E = cfg.hidden, len(layers), cfg.experts
    blocks = []
    for l, L in enumerate(layers):
        gen = torch.Generator().manual_seed(cfg.seed * 1000 + l)
        perm = torch.randperm(E, generator=gen).cuda()  # slot -> expert
        slot_of = torch.empty(E, dtype=torch.int32, device="cuda")
        slot_of[perm] = torch.arange(E, dtype=torch.int32, device="cuda")
        Lp = copy.copy(L)
        Lp.gate_up = L.gate_up.map(lambda a: a.index_select(0, perm))
        Lp.down = L.down.map(lambda a: a.index_select(0, perm))
        Lp.slot_of_expert = slot_of
        blocks.append(ops.MoeBlock(Lp))
    x = c1_tokens_device(cfg, nL)
    y = torch.empty_like(x)
    ws = torch.empty(blocks[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")

    def step():
        for l in range(nL):
            blocks[l].forward(x[l], out=y[l], workspace=ws)
    step()
    torch.cuda.synchronize()
    missing = blocks[-1].trace(1, workspace=ws)["missing_slots"]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(W):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(K):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / K / nL * 1000
    credited = (cfg.top_k + 1) * cfg.page_bytes
    gbs = credited / (us * 1e-6) / 1e9
    out = {"workload": f"c1 decode B=1, routed arrays as compact pages (all {E} experts, permuted slots), "
                       f"graph of {nL} layers",
           "us_per_layer": round(us, 2), "tokens_per_s": round(1e6 / us, 1),
           "achieved_GBps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "missing_slots": int(missing)}
    log(f"paged decode: {json.dumps(out)}")
    del blocks, g, x, y, ws
    return out


def c1_tokens_device(cfg, n, step=17):
    from astronomical_amd import device_synthetic as DS
    return DS.make_tokens_device(cfg, n, step=step).reshape(n, 1, cfg.hidden)


def affine_router_decode(CF, DS, ops, torch, layers, K, W, bits=4):
    """c1 decode B=1 with an affine router (mlp.gate quantized to 4-bit g64, as the
    reference's certified checkpoints have it) through a graph of the same layers' experts:
    the decode kernels' quantized router row GEMV in place of the bf16 one."""
    import copy
    from astronomical_amd import synthetic as S
    cfg = CF.C1
    H, nL = cfg.hidden, len(layers)
    rcfg = S.router_config(cfg, bits)
    blocks = []
    for l, L in enumerate(layers):
        Lq = copy.copy(L)
        Lq.router_w = None
        Lq.router_q = DS.affine(rcfg, cfg.seed, f"L{l}/router_q{bits}", 1, cfg.experts, H)
        blocks.append(ops.MoeBlock(Lq))
    x = DS.make_tokens_device(cfg, nL, step=13).reshape(nL, 1, H)
    y = torch.empty_like(x)
    ws = torch.empty(blocks[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")

    def step():
        for l in range(nL):
            blocks[l].forward(x[l], out=y[l], workspace=ws)
    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(W):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(K):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / K / nL * 1000
    credited = (cfg.top_k + 1) * cfg.page_bytes
    gbs = credited / (us * 1e-6) / 1e9
    out = {"workload": f"c1 decode B=1, {bits}-bit g64 affine router, graph of {nL} layers",
           "us_per_layer": round(us, 2), "tokens_per_s": round(1e6 / us, 1),
           "achieved_GBps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "router_bytes_per_layer": int(cfg.experts * H * (bits / 8 + 4 / 64))}
    log(f"affine-router decode: {json.dumps(out)}")
    del blocks, g, x, y, ws
    return out


def decoder_step(CF, DS, ops, torch, blocks, K, W):
    """The decoder's feed-forward step around the block (residual add + RMS norm, block,
    residual add) on the c1 layers: decode B=1 through a graph of all the layers, 2048-token
    prefill on layer 0, the RMS norm kernel alone, and Laguna's sigmoid router on c2-sized
    logits."""
    cfg = CF.C1
    H, nL, dev = cfg.hidden, len(blocks), torch.device("cuda")
    w = DS.make_tokens_device(cfg, 1, step=7).reshape(H)  # a bf16 weight vector (values ~N(0,1))
    T2 = 2048
    ws = torch.empty(blocks[0].workspace_bytes(T2) + 3 * T2 * H * 2 + 1024, dtype=torch.uint8, device=dev)
    h = DS.make_tokens_device(cfg, nL, step=3).reshape(nL, 1, H)
    a = DS.make_tokens_device(cfg, nL, step=4).reshape(nL, 1, H)
    outs = torch.empty_like(h)

    def step():
        for l in range(nL):
            blocks[l].decoder_feed_forward(h[l], w, 1e-6, attention_out=a[l], out=outs[l], workspace=ws)
    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(W):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(K):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    dec_us = e0.elapsed_time(e1) / K / nL * 1000

    def timed(fn, iters=10):
        """device time of fn, replayed from a graph of `iters` calls (no host launch cost)"""
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(iters):
                fn()
        gr.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        gr.replay()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / iters * 1000

    xp = DS.make_tokens_device(CF.C2, T2)
    ap = DS.make_tokens_device(CF.C2, T2, step=5)
    yp = torch.empty_like(xp)
    rp = torch.empty_like(xp)
    pre_us = timed(lambda: blocks[0].decoder_feed_forward(xp, w, 1e-6, attention_out=ap, out=yp, workspace=ws))
    rms_us = timed(lambda: ops.rms_norm(xp, w, 1e-6, attention_out=ap, residual_out=rp), 20)
    rms_bytes = 4 * T2 * H * 2  # read h and a, write r and n
    logits = DS.make_tokens_device(CF.C2, T2, step=6)[:, :cfg.experts].contiguous()
    bias = torch.zeros(cfg.experts, dtype=torch.float32, device=dev)
    lag_us = timed(lambda: ops.route_laguna_experts(logits, cfg.top_k, bias, 0.0, True), 20)
    return {"decoder_ffn_step": {
        "workload": f"c1 residual add + RMS norm + MoE block + residual add: decode B=1 through a graph of {nL} "
                    f"layers, and {T2}-token prefill on one layer",
        "decode_us_per_layer": round(dec_us, 2), "decode_tokens_per_s": round(1e6 / dec_us, 1),
        "prefill_us": round(pre_us, 1),
        "rms_norm_us_2048": round(rms_us, 2), "rms_norm_GBps": round(rms_bytes / (rms_us * 1e-6) / 1e9, 1)},
        "laguna_route": {"workload": f"Laguna sigmoid router, {T2} tokens x {cfg.experts} experts, top-{cfg.top_k}, "
                                     "correction bias, normalised", "us": round(lag_us, 2)}}


def page_load(CF, torch, L, n_experts=16, ids=(1, 3, 4, 6, 8, 10, 12, 15), reps=5):
    """Loads 8 experts of a c1-shaped checkpoint (the first 16 experts of layer 0, gate / up /
    down in two shards) from the page cache into HBM through 64 MiB of pinned staging."""
    import tempfile
    from safetensors.torch import save_file
    from astronomical_amd import pages as PG
    I = CF.C1.intermediate
    pre = "model.layers.0.mlp"

    def t(a):  # device int32 / bf16 -> host tensors safetensors writes as U32 / BF16
        a = a.detach().cpu().contiguous()
        return a.view(torch.uint32) if a.dtype == torch.int32 else a

    gu, dn = L.gate_up, L.down
    parts = {"gate_proj": [gu.w[:n_experts, :I], gu.scales[:n_experts, :I], gu.biases[:n_experts, :I]],
             "up_proj": [gu.w[:n_experts, I:], gu.scales[:n_experts, I:], gu.biases[:n_experts, I:]],
             "down_proj": [dn.w[:n_experts], dn.scales[:n_experts], dn.biases[:n_experts]]}
    with tempfile.TemporaryDirectory() as td:
        wm = {}
        for shard, projs in (("model-00001-of-00002.safetensors", ["gate_proj"]),
                             ("model-00002-of-00002.safetensors", ["up_proj", "down_proj"])):
            tensors = {f"{pre}.switch_mlp.{pj}.{pa}": t(a) for pj in projs
                       for pa, a in zip(("weight", "scales", "biases"), parts[pj])}
            save_file(tensors, os.path.join(td, shard))
            wm.update({k: shard for k in tensors})
        plan = PG.build_quantized_expert_layer_plan(td, wm, pre, CF.C1.bits, CF.C1.group_size)
        staging = torch.empty(64 << 20, dtype=torch.uint8).pin_memory()
        PG.load_quantized_expert_page(plan, ids, "cuda", staging=staging)  # page cache warm
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            page = PG.load_quantized_expert_page(plan, ids, "cuda", staging=staging)
            times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    return {"workload": f"c1 decode page: {len(ids)} of {n_experts} experts (gate, up, down: codes, "
                        "scales, biases) from a two-shard safetensors checkpoint in the page cache into HBM",
            "bytes": page.bytes_read, "ms": round(sec * 1e3, 3),
            "GBps": round(page.bytes_read / sec / 1e9, 2)}


def cpu_baseline(layer_dev, toks, cfg, xprefill, seconds):
    """The oracle (the C restatement of the reference's op graph, OpenMP over output rows) on the
    host cores: decode B=1 tokens/s on a bounded sample of the bench's own tokens, and a c2
    prefill sample (64 tokens, the sorted path), each the median of 5 runs, with every core this
    process may use and with one.  Cores: the process's CPU set, capped by OMP_NUM_THREADS when
    the environment sets it (the GPU box's share of its host)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import torch
    from astronomical_amd.ops import bf16_to_numpy, u32_to_numpy

    def host(a):
        return u32_to_numpy(a) if a.dtype == torch.int32 else bf16_to_numpy(a)
    Lh = layer_dev.map(host)
    avail = len(os.sched_getaffinity(0))
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    cores = min(avail, cap) if cap > 0 else avail
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    xs = bf16_to_numpy(toks.reshape(-1, cfg.hidden))
    xp = bf16_to_numpy(xprefill)
    per_run = seconds / 20.0  # 5 decode runs at each thread count take half the budget

    def decode_run():
        n, t0 = 0, time.perf_counter()
        while True:
            i = n % xs.shape[0]
            oracle.moe_block_forward(Lh, xs[i:i + 1])
            n += 1
            el = time.perf_counter() - t0
            if el >= per_run:
                return n / el

    def prefill_run(t):
        t0 = time.perf_counter()
        oracle.moe_block_forward(Lh, xp[:t])
        return t / (time.perf_counter() - t0)

    res = {}
    for name, threads, tp in (("all", cores, 64), ("one", 1, 16)):
        oracle.set_threads(threads)
        dec = statistics.median(decode_run() for _ in range(5))
        pre = statistics.median(prefill_run(tp) for _ in range(5))
        res[name] = {"threads": threads, "decode_tokens_per_s": round(dec, 2), "prefill_tokens": tp,
                     "prefill_tokens_per_s": round(pre, 2)}
    oracle.set_threads(cores)
    return {"value": res["all"]["decode_tokens_per_s"], "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"c1 decode B=1 through layer 0, median of 5 runs of {per_run:.1f} s each (oracle C "
                      f"restatement, OpenMP over output rows); prefill: c2 tokens through the sorted path",
            "nproc": os.cpu_count(), "affinity_cpus": avail, "cpu_model": model,
            "one_core": res["one"], "all_cores": res["all"]}


if __name__ == "__main__":
    main()
