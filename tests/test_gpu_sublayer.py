"""GPU parity of the RMS norms (kimi_linear/ops.rs:46-53, qwen38/ops.rs:25-33) and of the MoE
sublayer x += moe_forward(rmsnorm_1p(x, post_ln)) (qwen38/generate.rs:397-413) against the oracle.

Bars: the normalised rows bit-exact (the device's parallel fp64 sum of squares rounds to the same
fp32 mean square except within a few fp64 ulps of an fp32 boundary); sublayer expert ids bit-exact
and the MoE contribution (x_out - x) within 1e-5 relative L2.
"""
import numpy as np
import pytest

from helpers import bits_equal, normal, rel_l2

pytestmark = pytest.mark.gpu
RTOL = 1e-5


@pytest.mark.parametrize("n,s", [(4, 1), (6, 3), (6144, 2), (7168, 4), (8192, 8)])
@pytest.mark.parametrize("one_plus", [False, True])
def test_rmsnorm_rows_match_oracle(ctx, orc, n, s, one_plus):
    import torch
    v = normal((s, n), 7 * n + s, 3.0)
    w = normal(n, n + 1, 0.2)
    exp = (orc.rmsnorm_1p if one_plus else orc.rmsnorm)(v, w, 1e-6)
    dv = torch.from_numpy(v).cuda()
    ctx.rmsnorm(dv, torch.from_numpy(w).cuda(), s, n, 1e-6, one_plus=one_plus)
    assert bits_equal(dv.cpu().numpy(), exp)


def test_rmsnorm_kats_on_device(ctx, orc):
    # qwen38/ops.rs:42-52 and :73-81
    import torch
    v = torch.full((4,), 2.0, device="cuda")
    ctx.rmsnorm(v, torch.zeros(4, device="cuda"), 1, 4, 1e-6, one_plus=True)
    assert np.all(np.abs(v.cpu().numpy() - 1.0) < 1e-4)
    v = torch.full((8,), 3.0, device="cuda")
    ctx.rmsnorm(v, torch.full((8,), 0.05, device="cuda"), 1, 8, 1e-6, one_plus=True)
    assert abs(float(v[0]) - 1.05) < 1e-4


@pytest.mark.parametrize("name,ntok", [("c1", 1), ("c1", 2), ("c3", 1)])
def test_moe_sublayer_full_config(ctx, orc, name, ntok):
    import rabbit_amd.workloads as W
    from oracle.workload import HostLayer
    import torch
    cfg = W.CONFIGS[name]
    W.build_layer(ctx, cfg, layer=0, seed=1000)
    host = HostLayer(cfg, 1000)
    x = W.tokens(cfg, ntok, 1099)
    ln = normal(cfg.hidden, 31, 0.1)
    exp, eids, ew = host.sublayer(x, ln, 1e-6)
    k = cfg.topk
    dx = torch.from_numpy(x).cuda()
    ids = torch.empty(ntok * k, dtype=torch.int32, device="cuda")
    w = torch.empty(ntok * k, dtype=torch.float32, device="cuda")
    ctx.moe_sublayer(0, dx, ntok, torch.from_numpy(ln).cuda(), 1e-6, ids, w)
    got = dx.cpu().numpy().reshape(ntok, cfg.hidden)
    assert np.array_equal(ids.cpu().numpy().reshape(ntok, k), eids)
    assert rel_l2(w.cpu().numpy().reshape(ntok, k), ew) < RTOL
    assert rel_l2(got - x, exp - x) < RTOL


def test_moe_sublayer_host_buffers(ctx, orc):
    # the host-buffer entry point: same result as the device one on a small layer
    import rabbit_amd as R
    import torch
    H, I, E, k, S = 256, 128, 16, 4, 3
    experts = {}
    for e in range(E):
        g, u, d = orc.synth_mxfp4(I, H, 3 * e + 500), orc.synth_mxfp4(I, H, 3 * e + 501), orc.synth_mxfp4(H, I, 3 * e + 502)
        experts[e] = orc.Slot(e, d, gate=g, up=u)
        ctx.pool_put(0, R.Slot(e, R.QT.mxfp4(d.data, d.scale, H, I), gate=R.QT.mxfp4(g.data, g.scale, I, H),
                               up=R.QT.mxfp4(u.data, u.scale, I, H)))
    router = normal((E, H), 3, 0.05)
    ctx.moe_layer_set(0, R.FAMILY_QWEN38, H, I, E, k, router)
    L = orc.MoeLayer(orc.FAMILY_QWEN38, H, I, E, k, router, experts)
    x = normal((S, H), 4)
    ln = normal(H, 5, 0.1)
    exp, eids, _ = L.sublayer(x, S, ln, 1e-6)
    xh = x.copy()
    ids = np.empty(S * k, np.int32)
    ctx.moe_sublayer(0, xh, S, ln, 1e-6, ids)
    assert np.array_equal(ids.reshape(S, k), eids)
    assert rel_l2(xh - x, exp - x) < RTOL
    dx = torch.from_numpy(x).cuda()
    ctx.moe_sublayer(0, dx, S, torch.from_numpy(ln).cuda(), 1e-6)
    assert bits_equal(dx.cpu().numpy(), xh)


@pytest.mark.parametrize("name,ntok", [("c1", 1), ("c3", 1), ("c1", 2)])
def test_moe_sublayer_equals_its_composition(ctx, orc, name, ntok):
    """The sublayer (one token: the norm computed inside the router launch, the residual add in the
    down launch's store) equals its parts run one by one, bit for bit: rbt_rmsnorm_1p_d, then
    moe_forward on the normalised rows, then x + out."""
    import rabbit_amd.workloads as W
    import torch
    cfg = W.CONFIGS[name]
    W.build_layer(ctx, cfg, layer=0, seed=1000)
    H = cfg.hidden
    ln = torch.from_numpy(normal(H, 77, 0.1)).cuda()
    for seed in range(3):
        x = torch.from_numpy(W.tokens(cfg, ntok, 500 + seed)).cuda()
        nrm = x.clone()
        ctx.rmsnorm(nrm, ln, ntok, H, 1e-6, one_plus=True)
        out = torch.empty(ntok * H, dtype=torch.float32, device="cuda")
        ctx.moe_forward(0, nrm, ntok, out)
        exp = (x.reshape(-1) + out).cpu().numpy()
        got = x.clone()
        ctx.moe_sublayer(0, got, ntok, ln, 1e-6)
        assert bits_equal(got.cpu().numpy().ravel(), exp), seed
