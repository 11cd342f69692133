"""Wide parity sweep of the one-token decode (not collected by pytest: about 5 minutes on one MI355X).

Run from the repository root: `python tests/sweep_one_token.py`. For 1024 one-token calls at C2 and
at C1 and 256 of K3's latent MoE (then 256 two-token calls at C1 and 128 eight-token calls at C3, the
grouped decode): ids bit-exact against the oracle's sequential-fp32 routing, and
every token's output under the per-token rule of tests/test_gpu_moe.py (within 1e-5 relative L2 of
the oracle, or no farther from the fp64 truth than the oracle is); routing weights reported. Exits
non-zero on any id mismatch or rule failure."""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)
import torch, rabbit_amd as R, rabbit_amd.workloads as W
from oracle.workload import HostLayer, HostLatentLayer
from oracle import oracle as O
from helpers import rel_l2
from f64_truth import check_token, layer64
O.set_threads(16)
ctx = R.Context(0)

def sweep_moe(name, ntok, seed):
    t0 = time.time()
    cfg = W.CONFIGS[name]
    W.build_layer(ctx, cfg, layer=0, seed=1000)
    host = HostLayer(cfg, 1000)
    x = W.tokens(cfg, ntok, seed)
    xt = torch.from_numpy(x).cuda()
    out = torch.empty(ntok, cfg.hidden, device="cuda")
    ids = torch.empty(ntok, cfg.topk, dtype=torch.int32, device="cuda")
    w = torch.empty(ntok, cfg.topk, device="cuda")
    folded = []
    ctx.profile_read(reset=True)
    for t in range(ntok):
        ctx.moe_forward(0, xt[t:t + 1].contiguous(), 1, out[t], ids[t], w[t])
        if ctx.profile_read(reset=True)["ambiguous"]:
            folded.append(t)
    eids, ew = host.route(x)
    bad = np.where((ids.cpu().numpy() != eids).any(1))[0]
    got, gw = out.cpu().numpy(), w.cpu().numpy()
    worst, fails = 0.0, []
    for t in range(ntok):
        exp, _, _ = host.forward(x[t:t + 1])
        d = rel_l2(got[t], exp[0])
        worst = max(worst, d)
        if d >= 1e-5:
            truth = layer64(host, x[t:t + 1], eids[t:t + 1])
            _, eg, eo, ok = check_token(got[t], exp[0], truth[0], 1e-5)
            if not ok:
                fails.append((t, d, eg, eo, t in folded))
        if t % 256 == 255:
            print(f"  {name} {t + 1} tokens checked", flush=True)
    print(f"{name}: {ntok} tokens, folded {len(folded)}, id mismatches {len(bad)}, max rel l2 {worst:.2e}, "
          f"rule failures {len(fails)} {fails[:4]}, max |w| diff {np.abs(gw - ew).max():.2e}, {time.time() - t0:.0f} s",
          flush=True)
    return len(bad) == 0 and not fails

def sweep_k3(ntok, seed):
    t0 = time.time()
    cfg = W.CONFIGS["k3l"]
    lat = W.build_latent_layer(ctx, cfg, layer=0, seed=1000)
    host = HostLatentLayer(cfg, 1000)
    MH = cfg.extra["moe_hidden"]
    x = W.tokens(cfg, ntok, seed)
    xt = torch.from_numpy(x).cuda()
    out = torch.empty(ntok, cfg.hidden, device="cuda")
    ids = torch.empty(ntok, cfg.topk, dtype=torch.int32, device="cuda")
    w = torch.empty(ntok, cfg.topk, device="cuda")
    folded = []
    ctx.profile_read(reset=True)
    for t in range(ntok):
        ctx.latent_moe(0, MH, lat["down"], lat["up"], xt[t:t + 1].contiguous(), 1, out[t], norm=lat["norm"], eps=1e-5,
                       activation=lat["act"], ids_out=ids[t], w_out=w[t])
        if ctx.profile_read(reset=True)["ambiguous"]:
            folded.append(t)
    eids, ew = host.route(x)
    bad = np.where((ids.cpu().numpy() != eids).any(1))[0]
    got = out.cpu().numpy()
    worst, fails = 0.0, []
    for t in range(ntok):
        exp, _, _ = host.latent(x[t:t + 1])
        d = rel_l2(got[t], exp[0])
        worst = max(worst, d)
        if d >= 1e-5:
            fails.append((t, d, t in folded))
    print(f"k3l: {ntok} tokens, folded {len(folded)}, id mismatches {len(bad)}, max rel l2 {worst:.2e}, "
          f"over 1e-5 {len(fails)} {fails[:4]}, max |w| diff {np.abs(w.cpu().numpy() - ew).max():.2e}, "
          f"{time.time() - t0:.0f} s", flush=True)
    return len(bad) == 0

def sweep_batch(name, S, ncalls, seed):
    """Calls of S tokens (the grouped decode; the combine in unique_experts order): ids exact and
    every token under the per-token rule against the oracle's S-token call."""
    t0 = time.time()
    cfg = W.CONFIGS[name]
    W.build_layer(ctx, cfg, layer=0, seed=1000)
    host = HostLayer(cfg, 1000)
    x = W.tokens(cfg, S * ncalls, seed)
    xt = torch.from_numpy(x).cuda()
    out = torch.empty(S * ncalls, cfg.hidden, device="cuda")
    ids = torch.empty(S * ncalls, cfg.topk, dtype=torch.int32, device="cuda")
    w = torch.empty(S * ncalls, cfg.topk, device="cuda")
    for c in range(ncalls):
        sl = slice(c * S, (c + 1) * S)
        ctx.moe_forward(0, xt[sl].contiguous(), S, out[sl], ids[sl], w[sl])
    eids, ew = host.route(x)
    bad = np.where((ids.cpu().numpy() != eids).any(1))[0]
    got = out.cpu().numpy()
    worst, fails = 0.0, []
    for c in range(ncalls):
        sl = slice(c * S, (c + 1) * S)
        exp, _, _ = host.forward(x[sl])
        truth = None
        for i in range(S):
            t = c * S + i
            d = rel_l2(got[t], exp[i])
            worst = max(worst, d)
            if d >= 1e-5:
                if truth is None:
                    truth = layer64(host, x[sl], eids[sl])
                _, eg, eo, ok = check_token(got[t], exp[i], truth[i], 1e-5)
                if not ok:
                    fails.append((t, d, eg, eo))
    print(f"{name} S={S}: {ncalls} calls, id mismatches {len(bad)}, max rel l2 {worst:.2e}, rule failures "
          f"{len(fails)} {fails[:4]}, max |w| diff {np.abs(w.cpu().numpy() - ew).max():.2e}, {time.time() - t0:.0f} s",
          flush=True)
    return len(bad) == 0 and not fails


ok = sweep_moe("c2", 1024, 9001) & sweep_moe("c1", 1024, 9002) & sweep_k3(256, 9003)
ok = ok & sweep_batch("c1", 2, 256, 9004) & sweep_batch("c3", 8, 128, 9005)
sys.exit(0 if ok else 1)
