"""Benchmark: one MoE layer's batch-1 decode on one MI355X ("C1").

A step is one token through one Qwen3.8-shaped MoE layer: router logits over 512 experts, certified
top-10, the 10 routed MXFP4 SwiGLU experts plus the gated shared expert, ordered combine. All 512
experts (13.7 GB) are resident in HBM; every step feeds a different token, so the selected experts
rotate over the whole pool and the 256 MB Infinity Cache cannot serve them.

value    = microseconds per token (whole layer) over exactly --steps tokens, replayed through HIP
           graphs of at most --graph-tokens consecutive layer calls; every graph is launched once
           untimed first, so the timed launches are warm replays.
roofline = the dominant kernel (the most time per call): its algorithmic bytes per launch (the
           weight bytes of the experts it actually streamed) over its mean duration, measured live
           with HIP events that the kernel dispatch itself records (an eager pass after the timed
           one); traffic = its FETCH_SIZE + WRITE_SIZE bytes per launch from rocprofv3 counter runs
           (profiles/traffic_<config>.json, scaled by a plain copy's counters), when it is there.
cpu_baseline = the reference's AVX-512 (or AVX2; scalar for grouped int4, the reference's only
           tier) kernels restated in oracle/, timed on this host's cores over a bounded sample of
           the same tokens, warm (experts just generated) and cold (a 256 MiB eviction first).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config c1]

Other configurations (never the default line): c0 (one expert FFN, rbt_apply_single_expert_d), mm
(rbt_matmul_mxfp4_d at the reference's micro-benchmark shapes and C0's three matrices), c2 (GLM
grouped-int4 decode), c3 (K3 batch-8 Zipf decode), c4 (512-token prefill), k3l (K3's latent MoE),
c1s (the MoE sublayer: rmsnorm_1p, C1's layer, residual add).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer decode µs/token + expert GEMV HBM GB/s (% of 8 TB/s), MXFP4"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


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


def graph_time(hip, ctx, call, first, n, G):
    """Times calls call(first) .. call(first + n - 1) captured into HIP graphs of at most G calls.
    Each graph is launched once untimed (and synchronised) first; the timed region then launches
    every graph once. Returns (wall seconds, event milliseconds) of the timed region."""
    import torch
    graphs = []
    for g0 in range(first, first + n, G):
        g = Graph(hip, ctx.stream)
        g.begin()
        for t in range(g0, min(g0 + G, first + n)):
            call(t)
        g.end()
        graphs.append(g)
    for g in graphs:  # untimed first launch of every graph
        g.launch()
    ctx.sync()
    ext = ctx.torch_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(ext)
    for g in graphs:
        g.launch()
    ev1.record(ext)
    ctx.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = ev0.elapsed_time(ev1)
    for g in graphs:
        g.destroy()
    return wall, ev_ms


def kernel_table(ctx, run):
    """Per-kernel mean durations of the launches run() makes (eager, events recorded by each
    dispatch): {name: (launches, mean us)}."""
    ctx.sync()
    ctx.profile_kernels_read(reset=True)
    ctx.profile_kernels(True)
    try:
        run()
        ctx.sync()
    finally:
        ctx.profile_kernels(False)
    return ctx.profile_kernels_read(reset=True)


def kernel_role(name: str) -> str:
    """gateup / down / router / proj / other, from the kernel's (possibly mangled) name."""
    # k_xgemv1<NCH, KS, GU, PIN>: GU is the one-token expert's gate/up, PIN its down
    m = re.search(r"k_xgemv1ILi\d+ELi\d+ELb([01])ELb([01])E", name) or \
        re.search(r"k_xgemv1<\s*\d+,\s*\d+,\s*(true|false),\s*(true|false)", name)
    if m:
        gu, pin = m.group(1) in ("1", "true"), m.group(2) in ("1", "true")
        return "gateup" if gu else ("down" if pin else "other")
    if any(s in name for s in ("xgateup", "pgateup", "dgateup", "decode_gu_act", "gu1s_gemv")):
        return "gateup"
    if any(s in name for s in ("xdown", "pdown", "ddown", "down1c")):
        return "down"
    if "proj1" in name and "router" not in name:
        return "proj"
    m = re.search(r"k_decode_gemvILi\d+ELi\d+ELi\d+ELi(\d+)E", name) or \
        re.search(r"k_decode_gemv<\s*\d+,\s*\d+,\s*\d+,\s*(\d+)", name)
    if m:
        return {"0": "down", "1": "gateup", "2": "down", "3": "proj"}[m.group(1)]
    if "router" in name or "select" in name or "k_rcert" in name or "k_rcomb" in name:
        return "router"
    return "other"


def short_name(name: str) -> str:
    m = re.search(r"(k_[a-z0-9_]+)", name)
    return m.group(1) if m else name[:60]


def per_call(tab, ncalls):
    """{short name: [launches per call, mean us, us per call, role]} sorted by time per call."""
    rows = []
    for name, (launches, mean_us) in tab.items():
        rows.append((short_name(name), launches / ncalls, mean_us, launches * mean_us / ncalls, kernel_role(name),
                     name))
    rows.sort(key=lambda r: -r[3])
    return rows


def roofline(rows, role, bytes_per_launch, traffic_cfg, note=""):
    """The roofline object for the slowest kernel of `role` (rows from per_call)."""
    cand = [r for r in rows if r[4] == role]
    if not cand:
        return None
    r = cand[0]
    gbps = bytes_per_launch / (r[2] * 1e-6) / 1e9
    res = {"bound": "hbm", "kernel": r[0], "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
           "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes_per_launch": int(bytes_per_launch),
           "launch_us": round(r[2], 3), "traffic": traffic_of(traffic_cfg, r[5])}
    if note:
        res["note"] = note
    return res


def traffic_of(cfg_name, kernel_name):
    """FETCH_SIZE + WRITE_SIZE bytes per launch of `kernel_name` from profiles/traffic_<cfg>.json
    (written from two rocprofv3 --pmc runs of this benchmark), or None."""
    tf = os.path.join(ROOT, "profiles", f"traffic_{cfg_name}.json")
    try:
        t = json.load(open(tf))
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(short_name(kernel_name))
    return k.get("bytes_per_launch") if k else None


def kernels_json(rows):
    out = {}
    for r in rows:
        key = r[0] if r[0] not in out else f"{r[0]}[{r[4]}]"
        out[key] = {"per_call": round(r[1], 3), "mean_us": round(r[2], 3), "role": r[4]}
    return out


# ---- CPU baseline ------------------------------------------------------------------------------
def cpu_info() -> dict:
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except AttributeError:
        cpus = list(range(os.cpu_count() or 1))
    cores = set()
    for cpu in cpus:
        try:
            with open(f"/sys/devices/system/cpu/cpu{cpu}/topology/core_id") as f:
                core = f.read().strip()
            with open(f"/sys/devices/system/cpu/cpu{cpu}/topology/physical_package_id") as f:
                pkg = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            pass
    physical = len(cores) if cores else len(cpus)
    threads = physical
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        threads = min(threads, int(env))
    return {"model": model, "physical_cores": physical, "logical_cpus": len(cpus), "threads": max(1, threads)}


class Evictor:
    """256 MiB written before a cold call: the reference's cold benchmark evicts 64 MiB+
    (benches/kernels.rs:355-383); this host's last-level cache is smaller than 256 MiB."""

    def __init__(self):
        self.buf = np.ones(64 << 20, np.float32)

    def __call__(self):
        self.buf += 1.0


def simd_tier(O):
    L = O.lib()
    return "avx512" if L.orc_cpu_has_avx512() else ("avx2" if L.orc_cpu_has_avx2() else "scalar")


def cpu_line(us_warm, us_cold, unit, bytes_per_unit, info, kind, sample, extra=None):
    res = {"value": round(us_warm, 2), "unit": unit, "cores": info["threads"], "kind": kind, "sample": sample,
           "cold": round(us_cold, 2) if us_cold is not None else None,
           "gbps_warm": round(bytes_per_unit / (us_warm * 1e-6) / 1e9, 2),
           "gbps_cold": round(bytes_per_unit / (us_cold * 1e-6) / 1e9, 2) if us_cold else None,
           "cpu": info}
    if extra:
        res.update(extra)
    return res


def cpu_baseline_layer(cfg, seed, x_tokens, budget_s, gpu_out, bytes_per_token, simd=True, post_ln=None,
                       eps=1e-6):
    """The oracle's restated reference kernels on the same layer and tokens, one token per call.
    Experts the tokens route to are regenerated on the host first (not timed); each token runs warm
    (right after that) and cold (after an eviction). With post_ln: the MoE sublayer
    x + moe_forward(rmsnorm_1p(x, post_ln)) (qwen38/generate.rs:397-413)."""
    from oracle import oracle as O
    from oracle.workload import HostLayer
    info = cpu_info()
    O.set_threads(info["threads"])
    tier = simd_tier(O) if simd and cfg.kind == O.QT_MXFP4 else "scalar"
    host = HostLayer(cfg, seed)
    ev = Evictor()
    S = cfg.tokens
    warm, cold, outs, done = 0.0, 0.0, [], 0
    for t in range(0, x_tokens.shape[0], S):
        xt = x_tokens[t:t + S]
        if xt.shape[0] < S:
            break
        if post_ln is not None:
            from oracle import oracle as Oc
            ids, _ = host.route(np.stack([Oc.rmsnorm_1p(r, post_ln, eps) for r in xt]))
        else:
            ids, _ = host.route(xt)
        host.ensure(ids)
        lay = host._layer()
        run = (lambda: lay.sublayer(xt, S, post_ln, eps, simd=simd)[0]) if post_ln is not None else \
            (lambda: lay.forward(xt, S, simd=simd)[0])
        t0 = time.perf_counter()
        out = run()
        warm += time.perf_counter() - t0
        ev()
        t0 = time.perf_counter()
        run()
        cold += time.perf_counter() - t0
        outs.append(out)
        done += S
        if warm + cold >= budget_s and done >= 3 * S:
            break
        if len(host.experts) > 160:  # bound host memory (~4 GB of regenerated experts)
            host.experts.clear()
    per = lambda v: v / done * 1e6  # noqa: E731
    sample = (f"{done} tokens of {cfg.name} ({S} per call: {'rmsnorm_1p + ' if post_ln is not None else ''}"
              f"router + {cfg.topk} routed{' + shared' if cfg.shared else ''} experts"
              f"{' + residual' if post_ln is not None else ''}), {tier} tier of the reference's kernels restated "
              f"in C, rows in parallel on {info['threads']} threads")
    res = cpu_line(per(warm), per(cold), "us/token", bytes_per_token, info, "port", sample)
    g = gpu_out[:done].astype(np.float64).ravel()
    c = np.concatenate(outs).astype(np.float64).ravel()
    res["rel_l2_vs_gpu"] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    return res


# ---- layer configurations (c1, c2, c3) ---------------------------------------------------------
def expert_matrix_bytes(cfg, rows, cols):
    import rabbit_amd as R
    if cfg.kind == R.QT_MXFP4:
        return rows * cols // 2 + rows * cols // 32
    return rows * cols // 2 + rows * (cols // cfg.gs) * 4


def bench_layer(args, ctx, hip, cfg, pool_gb):
    """Decode configurations: one layer call of cfg.tokens tokens per graph node."""
    import torch
    import rabbit_amd.workloads as W
    S, H, I, k = cfg.tokens, cfg.hidden, cfg.inter, cfg.topk
    calls = max(1, args.steps // S) if S > 1 else args.steps
    steps = calls * S
    wcalls = max(1, args.warmup // S) if S > 1 else args.warmup
    ncalls = wcalls + calls
    x_all = torch.from_numpy(W.tokens(cfg, ncalls * S, args.seed + 5)).cuda()
    out_all = torch.empty_like(x_all)
    ids_all = torch.empty(ncalls * S * k, dtype=torch.int32, device="cuda")
    xs = [x_all[c * S:(c + 1) * S] for c in range(ncalls)]
    outs = [out_all[c * S:(c + 1) * S] for c in range(ncalls)]
    idv = [ids_all[c * S * k:(c + 1) * S * k] for c in range(ncalls)]

    def call(c):
        ctx.moe_forward(0, xs[c], S, outs[c], idv[c], sync=False)

    for c in range(wcalls):  # also sizes every scratch buffer, so capture allocates nothing
        call(c)
    ctx.sync()
    G = max(1, min(args.graph_tokens // S if S > 1 else args.graph_tokens, calls))
    wall, ev_ms = graph_time(hip, ctx, call, wcalls, calls, G)
    us_tok = wall / steps * 1e6
    log(f"[bench] {cfg.name}: timed {steps} tokens ({calls} calls): wall {wall * 1e3:.2f} ms "
        f"({us_tok:.2f} us/token), events {ev_ms:.2f} ms")

    # eager passes: the same calls without graphs (no profiling: the wall time per token, and the
    # host's time to issue them, C-ABI call through ctypes included), then per-kernel durations,
    # then the phase profile (streamed experts, exact folds)
    ctx.sync()
    t1 = time.perf_counter()
    for c in range(wcalls, ncalls):
        call(c)
    t_issue = time.perf_counter() - t1
    ctx.sync()
    eager_us = (time.perf_counter() - t1) / steps * 1e6
    issue_us = t_issue / calls * 1e6
    tab = kernel_table(ctx, lambda: [call(c) for c in range(wcalls, ncalls)])
    rows = per_call(tab, calls)
    ctx.profile_read(reset=True)
    ctx.profile_enable(True)
    for c in range(wcalls, ncalls):
        call(c)
    ctx.sync()
    prof = ctx.profile_read(reset=True)
    ctx.profile_enable(False)
    ids_np = ids_all.cpu().numpy().reshape(ncalls, S * k)[wcalls:]
    U = float(np.mean([len(np.unique(r[r >= 0])) for r in ids_np]))

    per_gu = 2 * expert_matrix_bytes(cfg, I, H)
    per_dn = expert_matrix_bytes(cfg, H, I)
    nsh = 1 if cfg.shared else 0
    n = max(1, prof["calls"])
    # experts each phase streamed: one token counts on the device what the gate/up launch streamed
    # (deferred decisions stream extra candidates; the shared expert's gate/up runs inside the
    # router launch); batches stream every unique expert plus the shared one
    if S == 1 and prof["gateup_experts"]:
        gu_exp, dn_exp = prof["gateup_experts"] / n, prof["down_experts"] / n
    else:
        gu_exp = dn_exp = U + nsh
    gu_bytes, dn_bytes = gu_exp * per_gu, dn_exp * per_dn
    rl = roofline(rows, "gateup", gu_bytes, args.config,
                  note=f"algorithmic bytes: gate+up weights of the {gu_exp:.2f} experts the kernel streams per call")
    gu = next((r for r in rows if r[4] == "gateup"), None)
    dn = next((r for r in rows if r[4] == "down"), None)
    ex = None
    if gu and dn:
        t_ex = gu[3] + dn[3]
        gb = (gu_bytes + dn_bytes) / (t_ex * 1e-6) / 1e9
        ex = {"bytes_per_call": int(gu_bytes + dn_bytes), "us_per_call": round(t_ex, 2), "gbps": round(gb, 1),
              "frac": round(gb / HBM_PEAK_GBPS, 4), "gateup_experts": round(gu_exp, 3),
              "down_experts": round(dn_exp, 3),
              "note": "the weight bytes the gate/up and down kernels stream over their own durations"}
    router_bytes = cfg.n_experts * H * 4 + (H * 4 if cfg.gated_shared else 0)
    call_bytes = (U + nsh) * (per_gu + per_dn) + router_bytes + 2 * S * H * 4
    call_gbps = call_bytes / (us_tok * S * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        ntok_cpu = min(x_all.shape[0] - wcalls * S, max(S, 64 if S == 1 else 4 * S))
        x0 = wcalls * S
        cpu = cpu_baseline_layer(cfg, args.seed, x_all[x0:x0 + ntok_cpu].cpu().numpy(), args.cpu_budget,
                                 out_all[x0:x0 + ntok_cpu].cpu().numpy(), call_bytes / S)
    import rabbit_amd as R
    res = {
        "metric": METRIC if args.config == "c1" else
        f"MoE-layer decode µs/token + expert GEMV HBM GB/s (% of 8 TB/s), {'MXFP4' if cfg.kind == R.QT_MXFP4 else 'grouped int4'}",
        "value": round(us_tok, 3), "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": wcalls * S,
        "ms_per_step": round(us_tok / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg.name, "hidden": H, "moe_inter": I, "n_experts": cfg.n_experts, "topk": k,
                   "shared_expert": cfg.shared, "weights": "mxfp4" if cfg.kind == R.QT_MXFP4 else f"int4-grouped gs{cfg.gs}",
                   "tokens_per_call": S, "resident_pool_gb": round(pool_gb, 2), "graph_calls": G,
                   "unique_experts_per_call": round(U, 2)},
        "roofline": rl,
        "expert_gemv": ex,
        "call": {"bytes_per_call": int(call_bytes), "us_per_call": round(us_tok * S, 2), "gbps": round(call_gbps, 1),
                 "frac": round(call_gbps / HBM_PEAK_GBPS, 4),
                 "note": "router + unique experts + shared expert + x/out over the whole call"},
        "kernels": kernels_json(rows),
        "eager_us_per_token": round(eager_us, 2),
        "host_issue_us_per_call": round(issue_us, 2),
        "router_exact_recomputes": int(prof["ambiguous"]),
        "cpu_baseline": cpu,
    }
    ctx.close()
    return res


# ---- prefill (c4) ------------------------------------------------------------------------------
def bench_prefill(args, ctx, hip, cfg, pool_gb):
    """C4: one MoE-layer call over cfg.tokens tokens (512) per step. value = us per layer call;
    roofline = the grouped gate/up GEMM (HBM: weights of every unique expert + shared; its MFMA
    utilisation beside it); the down GEMM is reported beside it."""
    import torch
    import rabbit_amd.workloads as W
    S, H, I, k = cfg.tokens, cfg.hidden, cfg.inter, cfg.topk
    steps = max(1, min(args.steps, 64))
    warm = max(1, min(args.warmup, 8))
    nb = steps + warm
    xs = [torch.from_numpy(W.tokens(cfg, S, args.seed + 5 + b)).cuda() for b in range(nb)]
    out = torch.empty(S * H, dtype=torch.float32, device="cuda")
    ids = torch.empty(nb, S * k, dtype=torch.int32, device="cuda")

    def call(b):
        ctx.moe_forward(0, xs[b], S, out, ids[b], sync=False)

    ctx.profile_read(reset=True)
    for b in range(warm):
        call(b)
    ctx.sync()
    amb = ctx.profile_read(reset=True)["ambiguous"] / warm  # exact folds of near-threshold experts
    wall, ev_ms = graph_time(hip, ctx, call, warm, steps, steps)
    us_call = wall / steps * 1e6
    log(f"[bench] prefill: {steps} calls of {S} tokens, {us_call:.1f} us/call (events {ev_ms / steps * 1e3:.1f})")
    tab = kernel_table(ctx, lambda: [call(b) for b in range(warm, nb)])
    rows = per_call(tab, steps)
    U = float(np.mean([len(np.unique(r)) for r in ids[warm:].cpu().numpy()]))
    nexp = U + 1  # + shared
    per_gu = 2 * I * (H // 2 + H // 32)
    per_dn = H * (I // 2 + I // 32)
    pairs = S * k + S
    gu_flops = 2.0 * pairs * 2 * I * H
    dn_flops = 2.0 * pairs * H * I
    rl = roofline(rows, "gateup", nexp * per_gu, "c4",
                  note=f"algorithmic bytes: gate+up weights of the {nexp:.1f} experts of the call, each read once")
    gu = next((r for r in rows if r[4] == "gateup"), None)
    dn = next((r for r in rows if r[4] == "down"), None)
    if rl and gu:
        rl["mfma_tflops"] = round(gu_flops / (gu[2] * 1e-6) / 1e12, 1)
        rl["mfma_util"] = round(gu_flops / (gu[2] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
    down = None
    if dn:
        down = {"kernel": dn[0], "bytes": int(nexp * per_dn), "us": round(dn[2], 2),
                "gbps": round(nexp * per_dn / (dn[2] * 1e-6) / 1e9, 1),
                "mfma_util": round(dn_flops / (dn[2] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
    cpu = None
    if not args.no_cpu:
        call(warm)  # the sampled call once more, its output kept for the comparison
        ctx.sync()
        cpu = cpu_baseline_prefill(cfg, args.seed, xs[warm].cpu().numpy(), nexp * (per_gu + per_dn),
                                   gpu_out=out.cpu().numpy())
    res = {
        "metric": "MoE-layer prefill us/call (512 tokens) + grouped-GEMM HBM GB/s and MFMA utilisation, MXFP4",
        "value": round(us_call, 1), "unit": "us/call", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(us_call / 1e3, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16-mfma/f32-acc", "data": "synthetic",
        "config": {"workload": cfg.name, "tokens_per_step": S, "hidden": H, "moe_inter": I,
                   "n_experts": cfg.n_experts, "topk": k, "shared_expert": cfg.shared, "weights": "mxfp4",
                   "resident_pool_gb": round(pool_gb, 2), "unique_experts_mean": round(U, 1)},
        "us_per_token": round(us_call / S, 3),
        "router_exact_recomputes": round(amb, 1),
        "roofline": rl,
        "down": down,
        "kernels": kernels_json(rows),
        "cpu_baseline": cpu,
    }
    ctx.close()
    return res


def cpu_baseline_prefill(cfg, seed, x, bytes_per_call, gpu_out=None):
    """The whole 512-token call on the host (the oracle's SIMD tier, the reference's order: every
    unique expert once over its tokens, the shared expert, the combine), experts generated first
    (not timed), warm (right after generation) and cold (256 MiB written first). gpu_out: the device
    output of the same call, for rel_l2_vs_gpu (bf16 prefill against the fp32 reference order)."""
    from oracle import oracle as O
    from oracle.workload import HostLayer
    info = cpu_info()
    O.set_threads(info["threads"])
    host = HostLayer(cfg, seed)
    S = x.shape[0]
    t0 = time.perf_counter()
    ids, _ = host.route(x)
    host.ensure(ids)
    gen_s = time.perf_counter() - t0
    lay = host._layer()
    t0 = time.perf_counter()
    out, _, _ = lay.forward(x, S, simd=True)
    us = (time.perf_counter() - t0) * 1e6
    Evictor()()  # cold: 256 MiB written first (the reference's cold benchmark, benches/kernels.rs:355-383)
    t0 = time.perf_counter()
    lay.forward(x, S, simd=True)
    us_cold = (time.perf_counter() - t0) * 1e6
    log(f"[bench] cpu prefill: {us / 1e3:.0f} ms per call warm, {us_cold / 1e3:.0f} cold "
        f"({len(host.experts)} experts generated in {gen_s:.0f} s)")
    res = cpu_line(us, us_cold, "us/call", bytes_per_call, info, "port",
                   f"one {S}-token call of {cfg.name} ({len(host.experts)} unique experts + shared), warm and "
                   f"cold, {simd_tier(O)} tier of the reference's matmul_mxfp4 restated in C, rows in parallel on "
                   f"{info['threads']} threads")
    if gpu_out is not None:
        g = np.asarray(gpu_out, np.float64).ravel()
        c = np.asarray(out, np.float64).ravel()
        res["rel_l2_vs_gpu"] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    return res


# ---- one expert (c0) and bare matrices (mm) ------------------------------------------------------
def rotating_pool(ctx, cfg, n, seed):
    """n C0-shaped experts in the pool of layer 0 (n x 26.7 MB, past the 256 MB Infinity Cache)."""
    import rabbit_amd.workloads as W
    H, I = cfg.hidden, cfg.inter
    for e in range(n):
        p = ctx.pool_alloc(0, e, cfg.kind, H, I, cfg.gs)
        s = p.contents
        for m, q in enumerate((s.gate, s.up, s.down)):
            W._synth(ctx, cfg.kind, q.data, q.scale, q.rows, q.cols, W.tensor_seed(seed, e, m), cfg)
    ctx.sync()


def bench_c0(args, ctx, hip, cfg):
    """C0: one MXFP4 SwiGLU expert FFN for one token (apply_single_expert, glm52/moe.rs:463), each
    call on another of 96 resident experts (2.6 GB) so the weights stream from HBM."""
    import torch
    import rabbit_amd as R
    import rabbit_amd.workloads as W
    from oracle import oracle as O
    from oracle.workload import host_expert
    H, I = cfg.hidden, cfg.inter
    NE = 96
    rotating_pool(ctx, cfg, NE, args.seed)
    slots = [ctx.pool_get(0, e) for e in range(NE)]
    steps, warm = args.steps, args.warmup
    ntok = steps + warm
    x_all = torch.from_numpy(W.tokens(cfg, ntok, args.seed + 5)).cuda()
    out_all = torch.zeros_like(x_all)
    w1 = torch.ones(1, dtype=torch.float32, device="cuda")
    # each call routes its one token to the slot it runs (ids = the slot's expert id)
    ids_per = torch.tensor([slots[e].contents.eid for e in range(NE)], dtype=torch.int32, device="cuda")

    def call(t):
        s = slots[t % NE].contents
        ctx.check(ctx.lib.rbt_apply_single_expert_d(ctx.h, C.byref(s), R._ptr(ids_per[t % NE:t % NE + 1]),
                                                    R._ptr(w1), 1, 1, R._ptr(x_all[t]), H, I, 0,
                                                    R._ptr(out_all[t])))

    ctx._torch_sync()
    for t in range(warm):
        call(t)
    ctx.sync()
    G = max(1, min(args.graph_tokens, steps))
    wall, ev_ms = graph_time(hip, ctx, call, warm, steps, G)
    us = wall / steps * 1e6
    out_all.zero_()
    torch.cuda.synchronize()
    tab = kernel_table(ctx, lambda: [call(t) for t in range(warm, ntok)])
    rows = per_call(tab, steps)
    per_gu = 2 * expert_matrix_bytes(cfg, I, H)
    per_dn = expert_matrix_bytes(cfg, H, I)
    rl = roofline(rows, "gateup", per_gu, "c0", note="gate+up weights of the one expert")
    ex_bytes = per_gu + per_dn
    gb = (ex_bytes + 2 * H * 4) / (us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        info = cpu_info()
        O.set_threads(info["threads"])
        ev = Evictor()
        warm_s = cold_s = 0.0
        n = 0
        outs = []
        for t in range(warm, min(ntok, warm + 16)):
            sl = host_expert(cfg, args.seed, t % NE)
            xt = x_all[t].cpu().numpy().reshape(1, H)
            o = np.zeros(H, np.float32)
            t0 = time.perf_counter()
            O.apply_single_expert(sl, np.array([[t % NE]], np.int32), np.ones((1, 1), np.float32), xt, H, I, o,
                                  simd=True)
            warm_s += time.perf_counter() - t0
            ev()
            o2 = np.zeros(H, np.float32)
            t0 = time.perf_counter()
            O.apply_single_expert(sl, np.array([[t % NE]], np.int32), np.ones((1, 1), np.float32), xt, H, I, o2,
                                  simd=True)
            cold_s += time.perf_counter() - t0
            outs.append(o)
            n += 1
        cpu = cpu_line(warm_s / n * 1e6, cold_s / n * 1e6, "us/call", ex_bytes, info, "port",
                       f"{n} calls of one C0 expert (gate, up, silu*up, down) for one token, {simd_tier(O)} tier "
                       f"of the reference's matmul_mxfp4 restated in C on {info['threads']} threads")
        g = out_all[warm:warm + n].cpu().numpy().astype(np.float64).ravel()
        c = np.stack(outs).astype(np.float64).ravel()
        cpu["rel_l2_vs_gpu"] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    res = {
        "metric": "Single-expert decode µs/call + HBM GB/s (% of 8 TB/s), MXFP4 (apply_single_expert, 1 token)",
        "value": round(us, 3), "unit": "us/call", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg.name, "hidden": H, "moe_inter": I, "weights": "mxfp4", "rotating_experts": NE,
                   "graph_calls": G},
        "roofline": rl,
        "call": {"bytes_per_call": ex_bytes + 2 * H * 4, "gbps": round(gb, 1), "frac": round(gb / HBM_PEAK_GBPS, 4)},
        "kernels": kernels_json(rows),
        "cpu_baseline": cpu,
    }
    ctx.close()
    return res


def bench_mm(args, ctx, hip):
    """rbt_matmul_mxfp4_d (matmul_mxfp4, kernels.rs:233) for one token at the reference's own
    micro-benchmark shapes (benches/kernels.rs:209-240,310-343: I = O = 4096, and K3's I = 3584,
    O = 3072) and C0's three matrices. GPU: each call on another of enough matrices to pass the
    256 MB Infinity Cache ("rotating"), and on one matrix over and over ("same": cache-resident).
    CPU: the reference's AVX-512 tier restated, warm (same matrix) and cold (256 MiB evicted)."""
    import torch
    import rabbit_amd as R
    from oracle import oracle as O
    shapes = [("k3_3584x3072", 3584, 3072), ("ref_4096x4096", 4096, 4096), ("c0_gate_8192x2048", 8192, 2048),
              ("c0_down_2048x8192", 2048, 8192)]
    info = cpu_info()
    O.set_threads(info["threads"])
    ev = Evictor()
    out = []
    steps = max(16, args.steps)
    for name, I, Ow in shapes:
        nbytes = Ow * (I // 2 + I // 32)
        nm = max(8, int(np.ceil(768e6 / nbytes)))
        data = torch.empty(nm, Ow * I // 2, dtype=torch.uint8, device="cuda")
        scale = torch.empty(nm, Ow * I // 32, dtype=torch.uint8, device="cuda")
        for m in range(nm):
            ctx.synth_mxfp4(data[m].data_ptr(), scale[m].data_ptr(), Ow, I, 77 + m)
        x = torch.from_numpy(np.random.default_rng(3).standard_normal((steps, I)).astype(np.float32)).cuda()
        y = torch.empty(steps, Ow, device="cuda")
        ctx.sync()

        def call_rot(t):
            ctx.check(ctx.lib.rbt_matmul_mxfp4_d(ctx.h, R._ptr(y[t]), R._ptr(x[t]), R._ptr(data[t % nm]),
                                                 R._ptr(scale[t % nm]), 1, I, Ow))

        def call_same(t):
            ctx.check(ctx.lib.rbt_matmul_mxfp4_d(ctx.h, R._ptr(y[t]), R._ptr(x[t]), R._ptr(data[0]),
                                                 R._ptr(scale[0]), 1, I, Ow))

        for t in range(4):
            call_rot(t)
        ctx.sync()
        G = min(args.graph_tokens, steps)
        w_rot, _ = graph_time(hip, ctx, call_rot, 0, steps, G)
        w_same, _ = graph_time(hip, ctx, call_same, 0, steps, G)
        us_rot, us_same = w_rot / steps * 1e6, w_same / steps * 1e6
        tab = kernel_table(ctx, lambda: [call_rot(t) for t in range(steps)])
        rows = per_call(tab, steps)
        k = rows[0]
        kgb = nbytes / (k[2] * 1e-6) / 1e9
        # CPU: matrix 0 on the host, warm (repeated) and cold (evicted before each call)
        hq = O.synth_mxfp4(Ow, I, 77)
        xh = x[0].cpu().numpy()
        reps = 20
        O.matmul_mxfp4_tier(xh, hq.data, hq.scale, 1, I, Ow)
        t0 = time.perf_counter()
        for _ in range(reps):
            O.matmul_mxfp4_tier(xh, hq.data, hq.scale, 1, I, Ow)
        cw = (time.perf_counter() - t0) / reps * 1e6
        cc = 0.0
        for _ in range(reps):
            ev()
            t0 = time.perf_counter()
            O.matmul_mxfp4_tier(xh, hq.data, hq.scale, 1, I, Ow)
            cc += time.perf_counter() - t0
        cc = cc / reps * 1e6
        yh = O.matmul_mxfp4_scalar(xh, hq.data, hq.scale, 1, I, Ow)
        ctx.check(ctx.lib.rbt_matmul_mxfp4_d(ctx.h, R._ptr(y[0]), R._ptr(x[0]), R._ptr(data[0]), R._ptr(scale[0]), 1,
                                             I, Ow))
        ctx.sync()
        yg = y[0].cpu().numpy()
        err = float(np.linalg.norm(yg.astype(np.float64) - yh) / np.linalg.norm(yh.astype(np.float64)))
        out.append({"shape": name, "i": I, "o": Ow, "bytes": nbytes,
                    "gpu_us_rotating": round(us_rot, 3), "gpu_us_same_matrix": round(us_same, 3),
                    "kernel": k[0], "kernel_us": round(k[2], 3), "kernel_gbps": round(kgb, 1),
                    "kernel_frac": round(kgb / HBM_PEAK_GBPS, 4),
                    "cpu_us_warm": round(cw, 1), "cpu_us_cold": round(cc, 1),
                    "cpu_gbps_warm": round(nbytes / (cw * 1e-6) / 1e9, 1), "rel_l2_vs_scalar": err})
        log(f"[bench] mm {name}: gpu {us_rot:.2f} us rotating / {us_same:.2f} same, kernel {k[2]:.2f} us "
            f"({kgb:.0f} GB/s); cpu {cw:.1f} warm / {cc:.1f} cold")
        del data, scale
        torch.cuda.empty_cache()
    head = out[0]
    res = {
        "metric": "matmul_mxfp4 µs/call (1 token) at the reference's micro-benchmark shapes, HBM GB/s",
        "value": head["gpu_us_rotating"], "unit": "us/call", "n_gpus": 1, "steps": steps, "warmup": 4,
        "ms_per_step": round(head["gpu_us_rotating"] / 1e3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "matmul_mxfp4_i3584_o3072", "shapes": [s[0] for s in shapes]},
        "roofline": {"bound": "hbm", "kernel": head["kernel"], "achieved": head["kernel_gbps"], "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": head["kernel_frac"], "bytes_per_launch": head["bytes"],
                     "launch_us": head["kernel_us"], "traffic": None},
        "shapes": out,
        "cpu_baseline": {"value": head["cpu_us_warm"], "unit": "us/call", "cores": info["threads"], "kind": "port",
                         "cold": head["cpu_us_cold"],
                         "sample": f"{reps} calls per shape on one matrix, the reference's {simd_tier(O)} tier "
                                   f"restated in C, rows in parallel on {info['threads']} threads; cold = 256 MiB "
                                   f"written before each call",
                         "cpu": info},
    }
    ctx.close()
    return res


# ---- K3 latent MoE (k3l) and the sublayer (c1s) -------------------------------------------------
def cpu_baseline_latent(cfg, seed, x_tokens, budget_s, gpu_out, bytes_per_token):
    """The oracle's SIMD tier on the latent workload (router, projections, routed experts, norm),
    experts regenerated on the host first (not timed)."""
    from oracle import oracle as O
    from oracle.workload import HostLatentLayer
    info = cpu_info()
    O.set_threads(info["threads"])
    host = HostLatentLayer(cfg, seed)
    ev = Evictor()
    warm, cold, outs, done = 0.0, 0.0, [], 0
    for t in range(x_tokens.shape[0]):
        xt = x_tokens[t:t + 1]
        ids, _ = host.route(xt)
        host.ensure(ids)
        lay = host._layer()

        def run():
            return lay.latent(xt, 1, host.mh, host.down, host.up, norm=host.norm, eps=1e-5, act=host.act, simd=True)

        t0 = time.perf_counter()
        out, _, _ = run()
        warm += time.perf_counter() - t0
        ev()
        t0 = time.perf_counter()
        run()
        cold += time.perf_counter() - t0
        outs.append(out)
        done += 1
        if warm + cold >= budget_s and done >= 3:
            break
        if len(host.experts) > 160:
            host.experts.clear()
    res = cpu_line(warm / done * 1e6, cold / done * 1e6, "us/token", bytes_per_token, info, "port",
                   f"{done} tokens of {cfg.name} (router + down projection + {cfg.topk} routed experts + norm + "
                   f"up projection), {simd_tier(O)} tier of the reference's matmul kernels restated in C, rows in "
                   f"parallel on {info['threads']} threads")
    g = gpu_out[:done].astype(np.float64).ravel()
    c = np.concatenate(outs).astype(np.float64).ravel()
    res["rel_l2_vs_gpu"] = float(np.linalg.norm(g - c) / np.linalg.norm(c))
    return res


def bench_latent(args, ctx, hip, cfg):
    """K3's latent MoE, one token per call (rbt_latent_moe_d), graph-replayed like the decode line.
    value = us per token; the call rate counts the router matrix, both projections and the routed
    experts' bytes once per token."""
    import torch
    import rabbit_amd.workloads as W
    t0 = time.perf_counter()
    lat = W.build_latent_layer(ctx, cfg, layer=0, seed=args.seed)
    pool_gb = ctx.pool_resident_bytes() / 1e9
    log(f"[bench] {cfg.name}: {cfg.n_experts} experts resident ({pool_gb:.2f} GB) in {time.perf_counter() - t0:.1f}s")
    H, MH, I, k, E = cfg.hidden, cfg.extra["moe_hidden"], cfg.inter, cfg.topk, cfg.n_experts
    steps, warm = args.steps, args.warmup
    ntok = steps + warm
    x_all = torch.from_numpy(W.tokens(cfg, ntok, args.seed + 5)).cuda()
    out_all = torch.empty_like(x_all)
    rows_x = [x_all[t] for t in range(ntok)]
    outs = [out_all[t] for t in range(ntok)]

    def call(t):
        ctx.latent_moe(0, MH, lat["down"], lat["up"], rows_x[t], 1, outs[t], norm=lat["norm"], eps=1e-5,
                       activation=lat["act"], sync=False)

    for t in range(warm):
        call(t)
    ctx.sync()
    G = max(1, min(args.graph_tokens, steps))
    wall, _ = graph_time(hip, ctx, call, warm, steps, G)
    us_per_token = wall / steps * 1e6
    tab = kernel_table(ctx, lambda: [call(t) for t in range(warm, ntok)])
    rows = per_call(tab, steps)
    log(f"[bench] timed {steps} tokens: {us_per_token:.2f} us/token")
    gs = cfg.extra["proj_gs"]
    per_exp = 2 * I * (MH // 2 + MH // 32) + MH * (I // 2 + I // 32)
    proj = 2 * (MH * H // 2 + MH * (H // gs) * 4)
    router = E * H * 4
    tok_bytes = k * per_exp + proj + router
    gbps = tok_bytes / (us_per_token * 1e-6) / 1e9
    rl = roofline(rows, "gateup", k * 2 * I * (MH // 2 + MH // 32), "k3l",
                  note=f"gate+up weights of the {k} routed experts")
    cpu = None
    if not args.no_cpu:
        n_cpu = min(8, steps)
        cpu = cpu_baseline_latent(cfg, args.seed, x_all[warm:warm + n_cpu].cpu().numpy(), args.cpu_budget,
                                  out_all[warm:warm + n_cpu].cpu().numpy(), tok_bytes)
    res = {
        "metric": "K3 latent-MoE decode us/token + effective HBM GB/s over the call (% of 8 TB/s), MXFP4 experts",
        "value": round(us_per_token, 3), "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(us_per_token / 1e3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg.name, "hidden": H, "moe_hidden": MH, "moe_inter": I, "n_experts": E, "topk": k,
                   "activation": "situ(4, 25)", "latent_norm": cfg.extra["latent_norm"],
                   "projections": f"int4-grouped gs{gs}", "tokens_per_step": 1,
                   "resident_pool_gb": round(pool_gb, 2), "graph_tokens": G},
        "roofline": rl,
        "call": {"bytes_per_token": tok_bytes, "gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
                 "note": "routed experts + router + both projections over the whole call"},
        "kernels": kernels_json(rows),
        "cpu_baseline": cpu,
    }
    ctx.close()
    return res


def bench_sublayer(args, ctx, hip, cfg):
    """The MoE half of a Qwen 3.8 decoder layer on C1's layer (rbt_moe_sublayer_d):
    x += moe_forward(rmsnorm_1p(x, post_ln)), one token per call, graph-replayed; the plain layer call
    is timed beside it in the same process, so the difference is the norm and the residual add."""
    import torch
    import rabbit_amd.workloads as W
    W.build_layer(ctx, cfg, layer=0, seed=args.seed)
    pool_gb = ctx.pool_resident_bytes() / 1e9
    steps, warm = args.steps, args.warmup
    ntok = steps + warm
    H = cfg.hidden
    x_all = torch.from_numpy(W.tokens(cfg, ntok, args.seed + 5)).cuda()
    out_all = torch.empty_like(x_all)
    ln = torch.from_numpy((np.random.default_rng(args.seed + 9).standard_normal(H) * 0.1).astype(np.float32)).cuda()
    rows_x = [x_all[t] for t in range(ntok)]
    outs = [out_all[t] for t in range(ntok)]
    G = max(1, min(args.graph_tokens, steps))

    def layer_call(t):
        ctx.moe_forward(0, rows_x[t], 1, outs[t], sync=False)

    def sub_call(t):
        ctx.moe_sublayer(0, rows_x[t], 1, ln, 1e-6, sync=False)

    for t in range(warm):  # sizes both calls' scratch, so capture allocates nothing
        layer_call(t)
        sub_call(t)
    ctx.sync()
    lw, _ = graph_time(hip, ctx, layer_call, warm, steps, G)
    sw, _ = graph_time(hip, ctx, sub_call, warm, steps, G)
    layer_us, sub_us = lw / steps * 1e6, sw / steps * 1e6
    log(f"[bench] sublayer {sub_us:.2f} us/token, layer alone {layer_us:.2f}")
    tab = kernel_table(ctx, lambda: [sub_call(t) for t in range(warm, ntok)])
    rows = per_call(tab, steps)
    gu_bytes = (cfg.topk + (1 if cfg.shared else 0)) * 2 * expert_matrix_bytes(cfg, cfg.inter, H)
    rl = roofline(rows, "gateup", gu_bytes, "c1",
                  note=f"algorithmic bytes: gate+up weights of the {cfg.topk} routed experts and the shared one")
    cpu = None
    if not args.no_cpu:
        # the CPU port on fresh copies of a few tokens, the device sublayer on the same copies
        ncpu = min(16, ntok)
        x0 = W.tokens(cfg, ncpu, args.seed + 77)
        xd = torch.from_numpy(x0.copy()).cuda()
        for t in range(ncpu):
            ctx.moe_sublayer(0, xd[t], 1, ln, 1e-6, sync=False)
        ctx.sync()
        bpt = (cfg.topk + (1 if cfg.shared else 0)) * 3 * expert_matrix_bytes(cfg, cfg.inter, H) + \
            (cfg.n_experts + 1) * H * 4
        cpu = cpu_baseline_layer(cfg, args.seed, x0, args.cpu_budget, xd.cpu().numpy(), bpt,
                                 post_ln=ln.cpu().numpy(), eps=1e-6)
    res = {
        "metric": "MoE sublayer decode us/token (rmsnorm_1p + MoE layer + residual add), MXFP4",
        "value": round(sub_us, 3), "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(sub_us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": cfg.name + "_sublayer", "hidden": H, "moe_inter": cfg.inter, "n_experts": cfg.n_experts,
                   "topk": cfg.topk, "shared_expert": cfg.shared, "weights": "mxfp4", "tokens_per_step": 1,
                   "resident_pool_gb": round(pool_gb, 2), "graph_tokens": G},
        "layer_us_per_token": round(layer_us, 3),
        "norm_and_residual_us": round(sub_us - layer_us, 3),
        "roofline": rl,
        "kernels": kernels_json(rows),
        "cpu_baseline": cpu,
    }
    ctx.close()
    return res


def bench_mix(args, ctx, hip):
    """Qwen 3.8's token mixers, one decode token per call: a Gated DeltaNet layer (128 V heads over 16
    K heads, 128 x 128 state per head, conv_dim 20480) and a GQA layer (64 query heads over 4 KV
    heads, head_dim 256) at context length args.context, each graph-replayed with its state carried.
    Roofline: the bytes each step must move (GDN: the state read and written plus the conv rows;
    GQA: the cached K and V rows read plus the new row written) over the step's duration."""
    import torch
    from oracle import oracle as O
    rng = np.random.default_rng(args.seed)
    steps, warm = args.steps, args.warmup
    # ---- GDN
    n_v, n_k, d_k, d_v, K = 128, 16, 128, 128, 4
    conv_dim = 2 * n_k * d_k + n_v * d_v
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    conv_w = f32(rng.standard_normal((conv_dim, K)) * 0.5)
    a_log, dt = f32(rng.standard_normal(n_v) * 0.5), f32(rng.standard_normal(n_v) * 0.5)
    nw = f32(1.0 + 0.1 * rng.standard_normal(d_v))
    conv_st = torch.zeros(conv_dim * (K - 1), dtype=torch.float32, device="cuda")
    states = torch.zeros(n_v * d_k * d_v, dtype=torch.float32, device="cuda")
    n = steps + warm
    xs = f32(rng.standard_normal((n, conv_dim)))
    zs = f32(rng.standard_normal((n, n_v * d_v)))
    As, Bs = f32(rng.standard_normal((n, n_v))), f32(rng.standard_normal((n, n_v)))
    out = torch.empty(n, n_v * d_v, dtype=torch.float32, device="cuda")

    def gdn_call(t):
        ctx.gdn_step(n_v, n_k, d_k, d_v, conv_w, a_log, dt, nw, 1e-6, conv_st, states, xs[t], zs[t], As[t], Bs[t],
                     out[t], kernel=K, sync=False)

    for t in range(warm):
        gdn_call(t)
    ctx.sync()
    G = max(1, min(args.graph_tokens, steps))
    wall, _ = graph_time(hip, ctx, gdn_call, warm, steps, G)
    gdn_us = wall / steps * 1e6
    tab = per_call(kernel_table(ctx, lambda: [gdn_call(t) for t in range(warm, n)]), steps)
    state_b = n_v * d_k * d_v * 4
    conv_b = conv_dim * (4 * K + 4 * (K - 1) * 2 + 4 + 4)  # weights, history read + written, x, output
    gdn_bytes = 2 * state_b + conv_b + 2 * n_v * d_v * 4
    head = next(r for r in tab if r[0] == "k_gdn_head")
    gdn_rl = {"bound": "hbm", "kernel": "k_gdn_head", "achieved": round(2 * state_b / (head[2] * 1e-6) / 1e9, 1),
              "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(2 * state_b / (head[2] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
              "bytes_per_launch": 2 * state_b, "launch_us": round(head[2], 3), "traffic": None,
              "note": "the heads' delta-rule states read and written once per token"}
    # ---- GQA
    nh, nkv, hd, rd = 64, 4, 256, 64
    T = args.context
    cap = T + steps + warm
    kc = f32(rng.standard_normal((cap, nkv * hd)))
    vc = f32(rng.standard_normal((cap, nkv * hd)))
    qn, kn = f32(0.1 * rng.standard_normal(hd)), f32(0.1 * rng.standard_normal(hd))
    qgs = f32(rng.standard_normal((n, 2 * nh * hd)))
    ks, vs = f32(rng.standard_normal((n, nkv * hd))), f32(rng.standard_normal((n, nkv * hd)))
    ctx_out = torch.empty(n, nh * hd, dtype=torch.float32, device="cuda")

    def gqa_call(t):
        ctx.gqa_step(nh, nkv, hd, rd, 1e7, 1.0 / 16.0, 1e-6, qn, kn, kc, vc, cap, T + t, qgs[t], ks[t], vs[t],
                     ctx_out[t], sync=False)

    for t in range(warm):
        gqa_call(t)
    ctx.sync()
    wall, _ = graph_time(hip, ctx, gqa_call, warm, steps, G)
    gqa_us = wall / steps * 1e6
    tab2 = per_call(kernel_table(ctx, lambda: [gqa_call(t) for t in range(warm, n)]), steps)
    kv_b = (T + warm + steps // 2) * nkv * hd * 4 * 2
    sc = next(r for r in tab2 if r[0] == "k_gqa_chunk")
    gqa_rl = {"bound": "hbm", "kernel": "k_gqa_chunk", "achieved": round(kv_b / (sc[2] * 1e-6) / 1e9, 1),
              "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(kv_b / (sc[2] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
              "bytes_per_launch": int(kv_b), "launch_us": round(sc[2], 3), "traffic": None,
              "note": f"the cached K and V rows of ~{T + warm + steps // 2} positions read once per token"}
    # ---- CPU: the oracle's restatement (scalar, one thread), a few tokens of each
    cpu = None
    if not args.no_cpu:
        info = cpu_info()
        st = O.GdnState(n_v, n_k, d_k, d_v, K)
        cw, al, dtn, nwn = (v.cpu().numpy() for v in (conv_w, a_log, dt, nw))
        xn, zn, an, bn = (v[:8].cpu().numpy() for v in (xs, zs, As, Bs))
        t0 = time.perf_counter()
        for t in range(8):
            O.gdn_step(st, xn[t], cw, zn[t], an[t], bn[t], al, dtn, nwn, 1e-6)
        g_cpu = (time.perf_counter() - t0) / 8 * 1e6
        kv = O.KvCache(nkv, hd, T + 4)
        kv.k[:T] = kc[:T].cpu().numpy()
        kv.v[:T] = vc[:T].cpu().numpy()
        kv.len = T
        qn_, kn_ = qn.cpu().numpy(), kn.cpu().numpy()
        t0 = time.perf_counter()
        for t in range(4):
            O.gqa_step(kv, qgs[t].cpu().numpy(), ks[t].cpu().numpy(), vs[t].cpu().numpy(), nh, qn_, kn_, 1e-6, rd, 1e7,
                       1.0 / 16.0)
        q_cpu = (time.perf_counter() - t0) / 4 * 1e6
        cpu = cpu_line(g_cpu + q_cpu, None, "us/token (one GDN + one GQA layer)", gdn_bytes + kv_b,
                       dict(info, threads=1), "port",
                       f"8 GDN tokens and 4 GQA tokens at context {T}, the oracle's scalar restatement",
                       {"gdn_us": round(g_cpu, 1), "gqa_us": round(q_cpu, 1)})
    res = {
        "metric": "Qwen 3.8 token mixers, decode us/token (one GDN layer + one GQA layer)",
        "value": round(gdn_us + gqa_us, 3), "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round((gdn_us + gqa_us) / 1e3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "qwen38_mixers", "gdn": f"{n_v}/{n_k} heads, {d_k}x{d_v} state, conv 4",
                   "gqa": f"{nh}/{nkv} heads x {hd}, rope {rd}", "context": T, "graph_tokens": G},
        "gdn_us": round(gdn_us, 3), "gqa_us": round(gqa_us, 3),
        "roofline": gdn_rl, "roofline_gqa": gqa_rl,
        "kernels": dict(kernels_json(tab), **kernels_json(tab2)),
        "cpu_baseline": cpu,
    }
    ctx.close()
    return res


def run_config(args, name, hip):
    """One configuration's result dict (its own context: the pool of one config at a time)."""
    import rabbit_amd as R
    import rabbit_amd.workloads as W
    ctx = R.Context(0)
    if name == "c1s":
        return bench_sublayer(args, ctx, hip, W.CONFIGS["c1"])
    if name == "mm":
        return bench_mm(args, ctx, hip)
    if name == "mix":
        return bench_mix(args, ctx, hip)
    cfg = W.CONFIGS[name]
    if name == "k3l":
        return bench_latent(args, ctx, hip, cfg)
    if name == "c0":
        return bench_c0(args, ctx, hip, cfg)
    t0 = time.perf_counter()
    W.build_layer(ctx, cfg, layer=0, seed=args.seed)
    pool_gb = ctx.pool_resident_bytes() / 1e9
    log(f"[bench] {cfg.name}: {cfg.n_experts} experts resident ({pool_gb:.2f} GB) in {time.perf_counter() - t0:.1f}s")
    if name == "c4":
        return bench_prefill(args, ctx, hip, cfg, pool_gb)
    return bench_layer(args, ctx, hip, cfg, pool_gb)


# The other BASELINE configurations, run after the headline line (C1) of a default run, each with a
# bounded step count of its own and a short CPU-baseline budget: (name, steps, warmup).
SUB_CONFIGS = [("c0", 128, 16), ("c2", 128, 16), ("c3", 128, 16), ("c4", 8, 2)]
SUB_KEYS = ("metric", "value", "unit", "steps", "warmup", "dtype", "config", "roofline", "expert_gemv", "call",
            "us_per_token", "down", "router_exact_recomputes", "cpu_baseline")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--config", default="c1", choices=["c0", "c1", "c2", "c3", "c4", "mm", "k3l", "c1s", "mix"])
    ap.add_argument("--context", type=int, default=4096, help="mix: GQA context length (cached positions)")
    ap.add_argument("--graph-tokens", type=int, default=64)
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU-baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sub", action="store_true",
                    help="c1: the headline line only (no c0/c2/c3/c4 sub-results)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run a 1 GiB device copy first (reference kernel for the FETCH/WRITE counters)")
    ap.add_argument("--seed", type=int, default=1000)
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (this build has no "
              "multi-GPU path: it measures one GPU's share of the layer at its real shape)", file=sys.stderr)
        sys.exit(2)

    import torch

    torch.zeros(1, device="cuda")
    if args.calibrate_copy:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        a.fill_(1.0)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b
    hip = hip_runtime()
    res = run_config(args, args.config, hip)
    if args.config == "c1" and not args.no_sub:
        # compact lines of the other configurations beside the headline (each its own pool)
        subs = {}
        for name, steps, warm in SUB_CONFIGS:
            t0 = time.perf_counter()
            sa = argparse.Namespace(**vars(args))
            sa.steps, sa.warmup, sa.cpu_budget = steps, warm, min(args.cpu_budget, 4.0)
            sa.config = name  # its own metric name and traffic file
            torch.cuda.empty_cache()
            r = run_config(sa, name, hip)
            subs[name] = {k: r[k] for k in SUB_KEYS if k in r}
            log(f"[bench] sub-result {name}: {r['value']} {r['unit']} ({time.perf_counter() - t0:.1f} s)")
        res["configs"] = subs
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
