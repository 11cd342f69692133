"""Benchmark: one MoE layer's batch-1 decode on one MI355X ("C1").

A step is one token through one Qwen3.8-shaped MoE layer: router logits over 512 experts, certified
top-10, the 10 routed MXFP4 SwiGLU experts plus the gated shared expert, ordered combine. All 512
experts (13.7 GB) are resident in HBM; every step feeds a different token, so the selected experts
rotate over the whole pool and the 256 MB Infinity Cache cannot serve them.

value    = microseconds per token (whole layer), timed over --steps tokens replayed through a HIP
           graph of --graph-tokens consecutive layer calls (the way a decode step would run).
roofline = the dominant kernel, the gate/up dequant-GEMV: algorithmic bytes per launch / its mean
           duration, measured live with HIP events on the library's stream (second pass; the events
           are recorded by the kernel dispatch itself, at its start and end).
cpu_baseline = the reference's AVX-512 (or AVX2) MXFP4 tier, restated in oracle/, timed on this
           host's cores over a bounded sample of the same tokens.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config c1]

--config c4 times the 512-token prefill instead, --config k3l Kimi K3's latent MoE (896 experts
at moe_hidden 3584, top-16, Situ, the routed-expert norm) one token per call, and --config c1s the
MoE sublayer (rmsnorm_1p, C1's layer, residual add); none of them is the default line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer decode µs/token + expert GEMV HBM GB/s (% of 8 TB/s), MXFP4"
HBM_PEAK_GBPS = 8000.0
# the gate/up kernel the MXFP4 decode path launches (its FETCH/WRITE counters: profiles/traffic_<cfg>.json)
ROOFLINE_KERNEL = "rbt::k_xgateup1f<16>"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def hip_runtime():
    return C.CDLL("libamdhip64.so.7")


class Graph:
    """hipGraph of work captured on one stream."""

    def __init__(self, hip, stream):
        self.hip, self.stream = hip, C.c_void_p(stream)
        self.graph, self.exec = C.c_void_p(), C.c_void_p()

    def begin(self):
        rc = self.hip.hipStreamBeginCapture(self.stream, 1)  # hipStreamCaptureModeThreadLocal
        if rc:
            raise RuntimeError(f"hipStreamBeginCapture -> {rc}")

    def end(self):
        rc = self.hip.hipStreamEndCapture(self.stream, C.byref(self.graph))
        if rc:
            raise RuntimeError(f"hipStreamEndCapture -> {rc}")
        rc = self.hip.hipGraphInstantiate(C.byref(self.exec), self.graph, None, None, C.c_size_t(0))
        if rc:
            raise RuntimeError(f"hipGraphInstantiate -> {rc}")

    def launch(self):
        rc = self.hip.hipGraphLaunch(self.exec, self.stream)
        if rc:
            raise RuntimeError(f"hipGraphLaunch -> {rc}")

    def destroy(self):
        if self.exec:
            self.hip.hipGraphExecDestroy(self.exec)
        if self.graph:
            self.hip.hipGraphDestroy(self.graph)


def physical_cores() -> int:
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    cores = set()
    try:
        for cpu in os.sched_getaffinity(0):
            with open(f"/sys/devices/system/cpu/cpu{cpu}/topology/core_id") as f:
                core = f.read().strip()
            with open(f"/sys/devices/system/cpu/cpu{cpu}/topology/physical_package_id") as f:
                pkg = f.read().strip()
            cores.add((pkg, core))
    except OSError:
        pass
    n = len(cores) if cores else avail
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        n = min(n, int(env))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, seed, x_tokens, budget_s, gpu_out=None):
    """Times the oracle's SIMD tier (the reference's AVX-512/AVX2 MXFP4 kernels, restated) on the
    same layer and tokens. Experts are regenerated on the host first (not timed)."""
    from oracle import oracle as O
    from oracle.workload import HostLayer
    threads = physical_cores()
    O.set_threads(threads)
    tier = "avx512" if O.lib().orc_cpu_has_avx512() else ("avx2" if O.lib().orc_cpu_has_avx2() else "scalar")
    host = HostLayer(cfg, seed)
    done, t_total, outs = 0, 0.0, []
    for t in range(x_tokens.shape[0]):
        xt = x_tokens[t:t + 1]
        ids, _ = host.route(xt)
        host.ensure(ids)
        t0 = time.perf_counter()
        out, _, _ = host._layer().forward(xt, 1, simd=True)
        t_total += time.perf_counter() - t0
        outs.append(out)
        done += 1
        if t_total >= budget_s and done >= 3:
            break
        if len(host.experts) > 160:  # bound host memory (~4 GB of regenerated experts)
            host.experts.clear()
    us = t_total / done * 1e6
    res = {"value": round(us, 1), "unit": "us/token", "cores": threads, "kind": "port",
           "sample": f"{done} tokens of {cfg.name} (router + {cfg.topk} routed + shared expert), "
                     f"{tier} tier of the reference's matmul_mxfp4 restated in C, rows in parallel "
                     f"on {threads} threads; {cpu_model()}"}
    if gpu_out is not None:
        g = gpu_out[:done].astype(np.float64).ravel()
        c = np.concatenate(outs).astype(np.float64).ravel()
        res["rel_l2_vs_gpu"] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    return res


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def bench_prefill(args, ctx, cfg, pool_gb):
    """C4: one MoE-layer call over cfg.tokens tokens (512) per step. value = us per layer call;
    roofline = the grouped gate/up GEMM (HBM: weights of every unique expert + shared; also its
    MFMA utilisation); the down GEMM is reported beside it."""
    import torch
    import rabbit_amd.workloads as W
    S, H, I, k = cfg.tokens, cfg.hidden, cfg.inter, cfg.topk
    steps = max(1, min(args.steps, 64))
    warm = max(1, min(args.warmup, 8))
    nb = steps + warm
    xs = [torch.from_numpy(W.tokens(cfg, S, args.seed + 5 + b)).cuda() for b in range(nb)]
    out = torch.empty(S * H, dtype=torch.float32, device="cuda")
    ids = torch.empty(S * k, dtype=torch.int32, device="cuda")
    uniq = []
    for b in range(warm):
        ctx.moe_forward(0, xs[b], S, out, ids, sync=False)
    ctx.sync()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for b in range(warm, nb):
        ctx.moe_forward(0, xs[b], S, out, ids, sync=False)
    ctx.sync()
    wall = time.perf_counter() - t0
    us_call = wall / steps * 1e6
    log(f"[bench] prefill: {steps} calls of {S} tokens, {us_call:.1f} us/call")
    ctx.profile_read(reset=True)
    ctx.profile_enable(True)
    for b in range(warm, nb):
        ctx.moe_forward(0, xs[b], S, out, ids, sync=False)
        ctx.sync()
        uniq.append(len(np.unique(ids.cpu().numpy())))
    prof = ctx.profile_read(reset=True)
    ctx.profile_enable(False)
    n = max(1, prof["calls"])
    gu_us = prof["gateup_ms"] / n * 1e3
    dn_us = prof["down_ms"] / n * 1e3
    rt_us = prof["router_ms"] / n * 1e3
    cb_us = prof["combine_ms"] / n * 1e3
    U = float(np.mean(uniq))
    nexp = U + 1  # + shared
    gu_bytes = nexp * 2 * I * (H // 2 + H // 32)
    dn_bytes = nexp * H * (I // 2 + I // 32)
    pairs = S * k + S
    gu_flops = 2.0 * pairs * 2 * I * H
    dn_flops = 2.0 * pairs * H * I
    gu_gbps = gu_bytes / (gu_us * 1e-6) / 1e9
    res = {
        "metric": "MoE-layer prefill us/call (512 tokens) + grouped-GEMM HBM GB/s and MFMA utilisation, MXFP4",
        "value": round(us_call, 1), "unit": "us/call", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(us_call / 1e3, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16-mfma/f32-acc", "data": "synthetic",
        "config": {"workload": cfg.name, "tokens_per_step": S, "hidden": H, "moe_inter": I,
                   "n_experts": cfg.n_experts, "topk": k, "shared_expert": cfg.shared, "weights": "mxfp4",
                   "resident_pool_gb": round(pool_gb, 2), "unique_experts_mean": round(U, 1)},
        "us_per_token": round(us_call / S, 3),
        "roofline": {"bound": "hbm", "kernel": "k_pgateup (grouped gate/up GEMM + SiLU)",
                     "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gu_gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": int(gu_bytes),
                     "launch_us": round(gu_us, 2), "traffic": None,
                     "mfma_tflops": round(gu_flops / (gu_us * 1e-6) / 1e12, 1),
                     "mfma_util": round(gu_flops / (gu_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
        "down": {"bytes": int(dn_bytes), "us": round(dn_us, 2), "gbps": round(dn_bytes / (dn_us * 1e-6) / 1e9, 1),
                 "mfma_util": round(dn_flops / (dn_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)},
        "phase_us": {"router+group": round(rt_us, 2), "gateup": round(gu_us, 2), "down": round(dn_us, 2),
                     "combine": round(cb_us, 2)},
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)
    ctx.close()


def cpu_baseline_latent(cfg, seed, x_tokens, budget_s, gpu_out=None):
    """The oracle's SIMD tier on the latent workload (router, projections, routed experts, norm),
    experts regenerated on the host first (not timed)."""
    from oracle import oracle as O
    from oracle.workload import HostLatentLayer
    threads = physical_cores()
    O.set_threads(threads)
    tier = "avx512" if O.lib().orc_cpu_has_avx512() else ("avx2" if O.lib().orc_cpu_has_avx2() else "scalar")
    host = HostLatentLayer(cfg, seed)
    done, t_total, outs = 0, 0.0, []
    for t in range(x_tokens.shape[0]):
        xt = x_tokens[t:t + 1]
        ids, _ = host.route(xt)
        host.ensure(ids)
        t0 = time.perf_counter()
        out, _, _ = host._layer().latent(xt, 1, host.mh, host.down, host.up, norm=host.norm, eps=1e-5,
                                         act=host.act, simd=True)
        t_total += time.perf_counter() - t0
        outs.append(out)
        done += 1
        if t_total >= budget_s and done >= 3:
            break
        if len(host.experts) > 160:
            host.experts.clear()
    us = t_total / done * 1e6
    res = {"value": round(us, 1), "unit": "us/token", "cores": threads, "kind": "port",
           "sample": f"{done} tokens of {cfg.name} (router + down projection + {cfg.topk} routed experts + norm + "
                     f"up projection), {tier} tier of the reference's matmul kernels restated in C, rows in "
                     f"parallel on {threads} threads; {cpu_model()}"}
    if gpu_out is not None:
        g = gpu_out[:done].astype(np.float64).ravel()
        c = np.concatenate(outs).astype(np.float64).ravel()
        res["rel_l2_vs_gpu"] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    return res


def bench_latent(args, ctx, hip, cfg):
    """K3's latent MoE, one token per call (rbt_latent_moe_d), timed as HIP-graph replays like the
    decode line. value = us per token; the effective rate counts the router matrix, both
    projections and the routed experts' bytes once per token."""
    import torch
    import rabbit_amd.workloads as W
    t0 = time.perf_counter()
    lat = W.build_latent_layer(ctx, cfg, layer=0, seed=args.seed)
    pool_gb = ctx.pool_resident_bytes() / 1e9
    log(f"[bench] {cfg.name}: {cfg.n_experts} experts resident ({pool_gb:.2f} GB) in {time.perf_counter() - t0:.1f}s")
    H, MH, I, k, E = cfg.hidden, cfg.extra["moe_hidden"], cfg.inter, cfg.topk, cfg.n_experts
    G = max(1, min(args.graph_tokens, args.steps))
    reps = (args.steps + G - 1) // G
    steps = reps * G
    ntok = steps + args.warmup
    x_all = torch.from_numpy(W.tokens(cfg, ntok, args.seed + 5)).cuda()
    out_all = torch.empty_like(x_all)
    rows = [x_all[t] for t in range(ntok)]
    outs = [out_all[t] for t in range(ntok)]

    def call(t):
        ctx.latent_moe(0, MH, lat["down"], lat["up"], rows[t], 1, outs[t], norm=lat["norm"], eps=1e-5,
                       activation=lat["act"], sync=False)

    for t in range(args.warmup):
        call(t)
    ctx.sync()
    graphs = []
    for r in range(reps):
        g = Graph(hip, ctx.stream)
        g.begin()
        for j in range(G):
            call(args.warmup + r * G + j)
        g.end()
        graphs.append(g)
    torch.cuda.synchronize()
    ctx.sync()
    t0 = time.perf_counter()
    for g in graphs:
        g.launch()
    ctx.sync()
    wall = time.perf_counter() - t0
    us_per_token = wall / steps * 1e6
    for g in graphs:
        g.destroy()
    t1 = time.perf_counter()
    for t in range(args.warmup, ntok):
        call(t)
    ctx.sync()
    eager_us = (time.perf_counter() - t1) / steps * 1e6
    log(f"[bench] timed {steps} tokens: {us_per_token:.2f} us/token (eager {eager_us:.2f})")

    gs = cfg.extra["proj_gs"]
    per_exp = 2 * I * (MH // 2 + MH // 32) + MH * (I // 2 + I // 32)
    proj = 2 * (MH * H // 2 + MH * (H // gs) * 4)
    router = E * H * 4
    tok_bytes = k * per_exp + proj + router
    gbps = tok_bytes / (us_per_token * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        n_cpu = min(8, ntok)
        cpu = cpu_baseline_latent(cfg, args.seed, x_all[:n_cpu].cpu().numpy(), args.cpu_budget,
                                  gpu_out=out_all[:n_cpu].cpu().numpy())
    res = {
        "metric": "K3 latent-MoE decode us/token + effective HBM GB/s over the call (% of 8 TB/s), MXFP4 experts",
        "value": round(us_per_token, 3), "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(us_per_token / 1e3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg.name, "hidden": H, "moe_hidden": MH, "moe_inter": I, "n_experts": E, "topk": k,
                   "activation": "situ(4, 25)", "latent_norm": cfg.extra["latent_norm"],
                   "projections": f"int4-grouped gs{gs}", "tokens_per_step": 1,
                   "resident_pool_gb": round(pool_gb, 2), "graph_tokens": G},
        "call_rate": {"bytes_per_token": tok_bytes, "gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
                      "note": "routed experts + router + both projections over the whole call; per-kernel "
                              "durations are in the rocprofv3 summary"},
        "eager_us_per_token": round(eager_us, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    ctx.close()


def graph_us_per_call(hip, ctx, call, ntok, warmup, G):
    """Warms up, then times graph replays of G consecutive calls call(t) over tokens warmup..ntok."""
    import torch
    for t in range(warmup):
        call(t)
    ctx.sync()
    steps = ntok - warmup
    graphs = []
    for r in range(steps // G):
        g = Graph(hip, ctx.stream)
        g.begin()
        for j in range(G):
            call(warmup + r * G + j)
        g.end()
        graphs.append(g)
    torch.cuda.synchronize()
    ctx.sync()
    t0 = time.perf_counter()
    for g in graphs:
        g.launch()
    ctx.sync()
    us = (time.perf_counter() - t0) / steps * 1e6
    for g in graphs:
        g.destroy()
    return us


def bench_sublayer(args, ctx, hip, cfg):
    """The MoE half of a Qwen 3.8 decoder layer on C1's layer (rbt_moe_sublayer_d):
    x += moe_forward(rmsnorm_1p(x, post_ln)), one token per call, graph-replayed; the plain layer call
    is timed beside it in the same process, so the difference is the norm and the residual add."""
    import torch
    import rabbit_amd.workloads as W
    W.build_layer(ctx, cfg, layer=0, seed=args.seed)
    pool_gb = ctx.pool_resident_bytes() / 1e9
    G = max(1, min(args.graph_tokens, args.steps))
    steps = ((args.steps + G - 1) // G) * G
    ntok = steps + args.warmup
    H = cfg.hidden
    x_all = torch.from_numpy(W.tokens(cfg, ntok, args.seed + 5)).cuda()
    out_all = torch.empty_like(x_all)
    ln = torch.from_numpy((np.random.default_rng(args.seed + 9).standard_normal(H) * 0.1).astype(np.float32)).cuda()
    rows = [x_all[t] for t in range(ntok)]
    outs = [out_all[t] for t in range(ntok)]
    layer_us = graph_us_per_call(hip, ctx, lambda t: ctx.moe_forward(0, rows[t], 1, outs[t], sync=False), ntok,
                                 args.warmup, G)
    sub_us = graph_us_per_call(hip, ctx, lambda t: ctx.moe_sublayer(0, rows[t], 1, ln, 1e-6, sync=False), ntok,
                               args.warmup, G)
    log(f"[bench] sublayer {sub_us:.2f} us/token, layer alone {layer_us:.2f}")
    res = {
        "metric": "MoE sublayer decode us/token (rmsnorm_1p + MoE layer + residual add), MXFP4",
        "value": round(sub_us, 3), "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(sub_us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg.name + "_sublayer", "hidden": H, "moe_inter": cfg.inter, "n_experts": cfg.n_experts,
                   "topk": cfg.topk, "shared_expert": cfg.shared, "weights": "mxfp4", "tokens_per_step": 1,
                   "resident_pool_gb": round(pool_gb, 2), "graph_tokens": G},
        "layer_us_per_token": round(layer_us, 3),
        "norm_and_residual_us": round(sub_us - layer_us, 3),
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)
    ctx.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--config", default="c1")
    ap.add_argument("--graph-tokens", type=int, default=64)
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU-baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run a 1 GiB device copy first (reference kernel for the FETCH/WRITE counters)")
    ap.add_argument("--seed", type=int, default=1000)
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (this build has no "
              "multi-GPU path: it measures one GPU's share of the layer at its real shape)", file=sys.stderr)
        sys.exit(2)

    import torch
    import rabbit_amd as R
    import rabbit_amd.workloads as W

    torch.zeros(1, device="cuda")
    if args.config == "c1s":
        return bench_sublayer(args, R.Context(0), hip_runtime(), W.CONFIGS["c1"])
    cfg = W.CONFIGS[args.config]
    if args.config == "k3l":
        ctx = R.Context(0)
        return bench_latent(args, ctx, hip_runtime(), cfg)
    if cfg.tokens != 1 and args.config != "c4":
        raise SystemExit(f"bench.py times batch-1 decode (c1) or the 512-token prefill (c4); {args.config} is a "
                         "parity-test configuration")
    ctx = R.Context(0)
    hip = hip_runtime()

    if args.calibrate_copy:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        a.fill_(1.0)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    t0 = time.perf_counter()
    W.build_layer(ctx, cfg, layer=0, seed=args.seed)
    pool_gb = ctx.pool_resident_bytes() / 1e9
    log(f"[bench] {cfg.name}: {cfg.n_experts} experts resident ({pool_gb:.2f} GB) in {time.perf_counter() - t0:.1f}s")
    if cfg.tokens != 1:
        return bench_prefill(args, ctx, cfg, pool_gb)

    G = max(1, min(args.graph_tokens, args.steps))
    reps = (args.steps + G - 1) // G
    steps = reps * G
    ntok = steps + args.warmup
    x_all = torch.from_numpy(W.tokens(cfg, ntok, args.seed + 5)).cuda()
    out_all = torch.empty_like(x_all)
    H = cfg.hidden
    rows = [x_all[t] for t in range(ntok)]
    outs = [out_all[t] for t in range(ntok)]

    # warmup (also sizes every scratch buffer, so capture allocates nothing)
    for t in range(args.warmup):
        ctx.moe_forward(0, rows[t], 1, outs[t], sync=False)
    ctx.sync()

    # --- pass 1: timed region, HIP-graph replay of G consecutive layer calls per launch ----------
    graphs = []
    for r in range(reps):
        g = Graph(hip, ctx.stream)
        g.begin()
        for j in range(G):
            t = args.warmup + r * G + j
            ctx.moe_forward(0, rows[t], 1, outs[t], sync=False)
        g.end()
        graphs.append(g)
    ext = ctx.torch_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ctx.sync()
    t0 = time.perf_counter()
    ev0.record(ext)
    for g in graphs:
        g.launch()
    ev1.record(ext)
    ctx.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = ev0.elapsed_time(ev1)
    us_per_token = wall / steps * 1e6
    log(f"[bench] timed {steps} tokens: wall {wall * 1e3:.2f} ms ({us_per_token:.2f} us/token), "
        f"events {ev_ms:.2f} ms")
    for g in graphs:
        g.destroy()

    # --- pass 2: per-phase kernel durations (HIP events on the library's stream) ----------------
    ctx.profile_read(reset=True)
    ctx.profile_enable(True)
    t1 = time.perf_counter()
    for t in range(args.warmup, ntok):
        ctx.moe_forward(0, rows[t], 1, outs[t], sync=False)
    ctx.sync()
    eager_us = (time.perf_counter() - t1) / steps * 1e6
    prof = ctx.profile_read(reset=True)
    ctx.profile_enable(False)
    n = max(1, prof["calls"])
    gu_us = prof["gateup_ms"] / n * 1e3
    dn_us = prof["down_ms"] / n * 1e3
    rt_us = prof["router_ms"] / n * 1e3
    cb_us = prof["combine_ms"] / n * 1e3

    nexp = cfg.topk + (1 if cfg.shared else 0)
    per_gu = 2 * cfg.inter * (H // 2 + H // 32)  # gate + up bytes of one expert
    per_dn = H * (cfg.inter // 2 + cfg.inter // 32)
    # experts each kernel actually streamed per call (the shared expert's gate/up may run inside the
    # router's selection launch, on the CUs it leaves idle)
    gu_exp = prof["gateup_experts"] / n if prof["gateup_experts"] else nexp
    dn_exp = prof["down_experts"] / n if prof["down_experts"] else nexp
    gu_bytes = int(round(gu_exp * per_gu))
    dn_bytes = int(round(dn_exp * per_dn))
    gu_gbps = gu_bytes / (gu_us * 1e-6) / 1e9
    # every expert's bytes over the time the layer spends in its expert kernels
    ex_bytes = nexp * (per_gu + per_dn)
    ex_gbps = ex_bytes / ((gu_us + dn_us) * 1e-6) / 1e9

    traffic = None
    tf = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tf):
        try:
            t = json.load(open(tf))
            # only a measurement of the kernel this build launches counts
            traffic = t.get("gateup_bytes_per_launch") if t.get("kernel") == ROOFLINE_KERNEL else None
        except (OSError, ValueError):
            traffic = None

    cpu = None
    if not args.no_cpu:
        n_cpu = min(64, ntok)
        cpu = cpu_baseline(cfg, args.seed, x_all[:n_cpu].cpu().numpy(), args.cpu_budget,
                           gpu_out=out_all[:n_cpu].cpu().numpy())

    res = {
        "metric": METRIC,
        "value": round(us_per_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_token / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg.name, "hidden": H, "moe_inter": cfg.inter, "n_experts": cfg.n_experts,
                   "topk": cfg.topk, "shared_expert": cfg.shared, "weights": "mxfp4" if cfg.kind == R.QT_MXFP4
                   else "int4-grouped", "tokens_per_step": 1, "resident_pool_gb": round(pool_gb, 2),
                   "graph_tokens": G},
        "roofline": {"bound": "hbm", "kernel": "k_xgateup1f (gate/up + SiLU, MFMA on fp4->bf16 weights, balanced over all CUs; settles deferred router decisions)",
                     "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gu_gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": gu_bytes,
                     "launch_us": round(gu_us, 2), "traffic": traffic},
        "expert_gemv": {"bytes_per_token": ex_bytes, "us": round(gu_us + dn_us, 2),
                        "gbps": round(ex_gbps, 1), "frac": round(ex_gbps / HBM_PEAK_GBPS, 4),
                        "experts": nexp, "gateup_kernel_experts": gu_exp, "down_kernel_experts": dn_exp,
                        "note": "all experts' bytes over the gate/up + down kernel times; experts the gate/up "
                                "kernel does not stream ran inside the router phase"},
        "phase_us": {"router": round(rt_us, 2), "gateup": round(gu_us, 2), "down": round(dn_us, 2),
                     "combine": round(cb_us, 2)},
        "eager_us_per_token": round(eager_us, 2),
        "router_exact_recomputes": int(prof["ambiguous"]),
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
