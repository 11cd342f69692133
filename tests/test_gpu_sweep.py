"""GPU parity of the one-token decode at the benchmark shapes over many tokens and the routing
corner cases (test_gpu_moe.py covers the layer kinds; this file covers breadth at full size).

* A reduced sweep: 64 one-token calls each at C1 (MXFP4, matrix cores) and C2 (grouped int4, the
  decode GEMVs): ids bit-exact, every token's output under the per-token rule (f64_truth.check_token:
  within 1e-5 relative L2 of the oracle, or, where the oracle's sequential fp32 sums are the ones
  off, no farther from the fp64 truth than the oracle and within 2e-5 of it), weights within 1e-5.
* Every key equal (x = 0, or a zero router): more than 64 candidates tie, so the selection inside the
  gate/up launch takes its general path in every workgroup; the winners are the k lowest ids (the
  reference's strict `>` scans keep the first of equal keys, qwen38/moe.rs:48-58,
  glm52/moe.rs:170-186).
* Five experts tied at the top-k boundary whose places only the exact folds decide
  (helpers.tied_boundary_router): the deferred decision streams k + 4 routed pairs.
* Kimi K3's latent MoE at its benchmark shape (896 experts, top-16, moe_hidden 3584, moe_inter
  3072, Situ(4, 25), the routed-expert norm; kimi_k3/moe.rs:64-116), including a folded boundary
  and a tied router.
"""
import numpy as np
import pytest

from helpers import rel_l2

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def _layer(ctx, name):
    import rabbit_amd.workloads as W
    from oracle.workload import HostLayer
    cfg = W.CONFIGS[name]
    info = W.build_layer(ctx, cfg, layer=0, seed=1000)
    return cfg, info, HostLayer(cfg, 1000)


def _reset_router(ctx, cfg, info, router):
    import torch
    t_gate = torch.from_numpy(info["shared_gate"]).cuda() if info["shared_gate"] is not None else None
    t_lb = torch.from_numpy(info["logit_bias"]).cuda() if info["logit_bias"] is not None else None
    ctx.moe_layer_set(0, cfg.family, cfg.hidden, cfg.inter, cfg.n_experts, cfg.topk, torch.from_numpy(router).cuda(),
                      shared=info["shared"], shared_gate=t_gate, logit_bias=t_lb, norm_topk=True, routed_scale=1.0)
    torch.cuda.synchronize()


def _one_token(ctx, cfg, x):
    import torch
    out = torch.empty(cfg.hidden, dtype=torch.float32, device="cuda")
    ids = torch.empty(cfg.topk, dtype=torch.int32, device="cuda")
    w = torch.empty(cfg.topk, dtype=torch.float32, device="cuda")
    ctx.moe_forward(0, torch.from_numpy(np.ascontiguousarray(x)).cuda(), 1, out, ids, w)
    return out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()


def _check_one(host, x, out, ids, w, tag):
    from f64_truth import check_token, layer64
    eids, ew = host.route(x)
    assert np.array_equal(ids, eids[0]), (tag, ids, eids[0])
    assert np.max(np.abs(w - ew[0])) < 1e-5, (tag, np.max(np.abs(w - ew[0])))
    exp, _, _ = host.forward(x)
    d = rel_l2(out, exp[0])
    if d < RTOL:
        return d
    truth = layer64(host, x, eids)
    d, eg, eo, ok = check_token(out, exp[0], truth[0], RTOL)
    assert ok, f"{tag}: device vs oracle {d:.3e}, device vs fp64 {eg:.3e}, oracle vs fp64 {eo:.3e}"
    return d


@pytest.mark.parametrize("name,seed", [("c1", 9002), ("c2", 9001)])
def test_one_token_sweep(ctx, orc, name, seed):
    import rabbit_amd.workloads as W
    import torch
    cfg, _, host = _layer(ctx, name)
    ntok = 64
    x = W.tokens(cfg, ntok, seed)
    xt = torch.from_numpy(x).cuda()
    out = torch.empty(ntok, cfg.hidden, device="cuda")
    ids = torch.empty(ntok, cfg.topk, dtype=torch.int32, device="cuda")
    w = torch.empty(ntok, cfg.topk, device="cuda")
    ctx.profile_read(reset=True)
    folded = 0
    for t in range(ntok):
        ctx.moe_forward(0, xt[t:t + 1].contiguous(), 1, out[t], ids[t], w[t])
        folded += bool(ctx.profile_read(reset=True)["ambiguous"])
    got, gi, gw = out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()
    worst = 0.0
    for t in range(ntok):
        worst = max(worst, _check_one(host, x[t:t + 1], got[t], gi[t], gw[t], f"{name} token {t}"))
    print(f"{name}: {ntok} one-token calls, {folded} with exact folds, largest device vs oracle {worst:.2e}")


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_one_token_all_keys_equal(ctx, orc, name):
    """x = 0 (every logit exactly 0), then a zero router with a random token: every key is equal,
    the winners are ids 0 .. k-1 in that order, and the output is the oracle's (zero for x = 0)."""
    import rabbit_amd.workloads as W
    cfg, info, host = _layer(ctx, name)
    k = cfg.topk
    x0 = np.zeros((1, cfg.hidden), np.float32)
    out, ids, w = _one_token(ctx, cfg, x0)
    assert list(ids) == list(range(k))
    _check_one(host, x0, out, ids, w, f"{name} x = 0")
    assert not np.any(out)
    router = np.zeros((cfg.n_experts, cfg.hidden), np.float32)
    _reset_router(ctx, cfg, info, router)
    host.router = router
    for t in range(2):
        x = W.tokens(cfg, 1, 31 + t)
        out, ids, w = _one_token(ctx, cfg, x)
        assert list(ids) == list(range(k))
        _check_one(host, x, out, ids, w, f"{name} zero router, token {t}")
        assert np.any(out)


@pytest.mark.parametrize("name", ["c1", "c2"])
def test_one_token_tied_boundary(ctx, orc, name):
    """Five experts tied at the last top-k place (helpers.tied_boundary_router): the deferred
    decision streams k + 4 routed pairs, workgroup 0 folds all five, and the highest id (ranked last
    by the midpoint order) wins."""
    import rabbit_amd.workloads as W
    from helpers import tied_boundary_router
    cfg, info, host = _layer(ctx, name)
    x = W.tokens(cfg, 1, 778)
    router, tied, _, hi = tied_boundary_router(cfg.n_experts, cfg.hidden, cfg.topk, x[0])
    _reset_router(ctx, cfg, info, router)
    host.router = router
    ctx.profile_read(reset=True)
    out, ids, w = _one_token(ctx, cfg, x)
    assert ctx.profile_read(reset=True)["ambiguous"], "the router decision did not need exact folds"
    assert sorted(ids) == sorted(hi + [tied[-1]])
    _check_one(host, x, out, ids, w, f"{name} tied boundary")


def _k3_bench(ctx):
    import rabbit_amd.workloads as W
    from oracle.workload import HostLatentLayer
    cfg = W.CONFIGS["k3l"]
    lat = W.build_latent_layer(ctx, cfg, layer=0, seed=1000)
    return cfg, lat, HostLatentLayer(cfg, 1000)


def _k3_call(ctx, cfg, lat, x):
    import torch
    MH = cfg.extra["moe_hidden"]
    S = x.shape[0]
    out = torch.empty(S, cfg.hidden, device="cuda")
    ids = torch.empty(S, cfg.topk, dtype=torch.int32, device="cuda")
    w = torch.empty(S, cfg.topk, device="cuda")
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    for t in range(S):  # one token per call: the one-token decode
        ctx.latent_moe(0, MH, lat["down"], lat["up"], xt[t:t + 1].contiguous(), 1, out[t], norm=lat["norm"],
                       eps=1e-5, activation=lat["act"], ids_out=ids[t], w_out=w[t])
    return out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()


def _k3_check(host, x, out, ids, w, tag):
    eids, ew = host.route(x)
    assert np.array_equal(ids, eids), tag
    assert np.max(np.abs(w - ew)) < 1e-5, (tag, np.max(np.abs(w - ew)))
    exp, _, _ = host.latent(x)
    worst = 0.0
    for t in range(x.shape[0]):
        d = rel_l2(out[t], exp[t])
        assert d < RTOL, (tag, t, d)
        worst = max(worst, d)
    return worst


def test_k3_latent_bench_shape(ctx, orc):
    """K3's latent MoE at the benchmark's shape, one token per call: 12 random tokens (some need exact
    folds), then a folded boundary at top-16 (five tied experts, 20 routed pairs streamed) and a
    zero router (every key equal: the general selection in every workgroup, ids 0..15)."""
    import rabbit_amd as R
    import torch
    import rabbit_amd.workloads as W
    from helpers import tied_boundary_router
    cfg, lat, host = _k3_bench(ctx)
    x = W.tokens(cfg, 12, 9003)
    ctx.profile_read(reset=True)
    out, ids, w = _k3_call(ctx, cfg, lat, x)
    folded = ctx.profile_read(reset=True)["ambiguous"]
    worst = _k3_check(host, x, out, ids, w, "random tokens")
    print(f"k3l: 12 tokens, {folded} exact folds, largest device vs oracle {worst:.2e}")
    # the correction bias off, so that the router alone decides
    zero_bias = np.zeros(cfg.n_experts, np.float32)
    xb = W.tokens(cfg, 1, 9004)
    router, tied, _, hi = tied_boundary_router(cfg.n_experts, cfg.hidden, cfg.topk, xb[0])
    for rt, xx, tag in ((router, xb, "tied boundary"), (np.zeros_like(router), W.tokens(cfg, 1, 9005), "zero router")):
        ctx.moe_layer_set(0, cfg.family, cfg.hidden, cfg.inter, cfg.n_experts, cfg.topk, torch.from_numpy(rt).cuda(),
                          router_bias=torch.from_numpy(zero_bias).cuda(), norm_topk=True, routed_scale=1.0)
        torch.cuda.synchronize()
        host.router, host.bias = rt, zero_bias
        ctx.profile_read(reset=True)
        out, ids, w = _k3_call(ctx, cfg, lat, xx)
        amb = ctx.profile_read(reset=True)["ambiguous"]
        if tag == "tied boundary":
            assert amb, "the router decision did not need exact folds"
            assert sorted(ids[0]) == sorted(hi + [tied[-1]])
        else:
            assert list(ids[0]) == list(range(cfg.topk))
        _k3_check(host, xx, out, ids, w, tag)
    assert R is not None
