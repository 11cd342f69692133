"""GPU parity of Kimi K3's additions on the expert path against the oracle: the Situ activation
(glm52/moe.rs:41-70) on single experts, and the latent MoE (kimi_k3/moe.rs:64-116): routing at full
width, experts at moe_hidden, the optional rmsnorm of the summed rows, the up projection.

Bars: expert ids bit-exact, routing weights and outputs within 1e-5 relative L2 (the device's tanhf
and expf differ from the host's by a few ulps; the sums run in another order).
"""
import numpy as np
import pytest

from helpers import bits_equal, normal, rel_l2

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def _dev_qt(R, q):
    import torch
    if q.kind == R.QT_MXFP4:
        return R.QT.mxfp4(torch.from_numpy(q.data).cuda(), torch.from_numpy(q.scale).cuda(), q.rows, q.cols)
    if q.kind == R.QT_I4_GROUPED:
        return R.QT.i4g(torch.from_numpy(q.data).cuda(), torch.from_numpy(q.scale).cuda(), q.rows, q.cols,
                        q.group_size)
    return R.QT.f32(torch.from_numpy(q.data).cuda(), q.rows, q.cols)


def _host_qt(R, q):
    if q.kind == R.QT_MXFP4:
        return R.QT.mxfp4(q.data, q.scale, q.rows, q.cols)
    if q.kind == R.QT_I4_GROUPED:
        return R.QT.i4g(q.data, q.scale, q.rows, q.cols, q.group_size)
    return R.QT.f32(q.data, q.rows, q.cols)


def _synth(orc, kind, rows, cols, seed):
    if kind == "i4g":
        return orc.synth_i4g(rows, cols, 16, seed)
    if kind == "i4g32":
        return orc.synth_i4g(rows, cols, 32, seed)
    return orc.synth_mxfp4(rows, cols, seed)


# x_std puts the gate dot products at O(1-10), where Situ and SiLU differ. Hidden 3584 takes the
# one-launch gate/up + activation kernel (MXFP4 and grouped int4 with group 32), 8192 the stacked
# GEMV and the activation kernel, 70 x 24 the generic per-pair kernel.
@pytest.mark.parametrize("kind,H,I,x_std", [("mxfp4", 8192, 2048, 0.5), ("mxfp4", 3584, 3072, 0.5),
                                            ("i4g32", 3584, 1024, 1.0), ("i4g", 70, 24, 20.0)])
@pytest.mark.parametrize("lb", [25.0, None])
def test_apply_single_expert_situ(ctx, orc, kind, H, I, x_std, lb):
    import rabbit_amd as R
    g, u, dn = _synth(orc, kind, I, H, 1), _synth(orc, kind, I, H, 2), _synth(orc, kind, H, I, 3)
    slot = orc.Slot(5, dn, gate=g, up=u)
    s, k = 3, 2
    x = normal((s, H), 7, x_std)
    ids = np.array([[5, 1], [2, 3], [0, 5]], np.int32)
    w = np.array([[0.6, 0.1], [1.0, 1.0], [0.2, -0.4]], np.float32)
    exp = orc.apply_single_expert(slot, ids, w, x, H, I, np.zeros(s * H, np.float32), act=orc.situ(4.0, lb))
    silu = orc.apply_single_expert(slot, ids, w, x, H, I, np.zeros(s * H, np.float32))
    assert rel_l2(exp, silu) > 1e-2  # the activation matters at these magnitudes
    rs = R.Slot(5, _host_qt(R, dn), gate=_host_qt(R, g), up=_host_qt(R, u))
    out = np.zeros(s * H, np.float32)
    ctx.apply_single_expert(rs, ids, w, s, k, x, H, I, out, activation=R.situ(4.0, lb))
    assert rel_l2(out, exp) < RTOL
    assert np.array_equal(out.reshape(s, H)[1], np.zeros(H, np.float32))  # token 1 did not pick expert 5
    # device buffers, and the fused gate_up layout (bit-exact with separate, glm52/moe.rs:885-919)
    import torch
    ds = R.Slot(5, _dev_qt(R, dn), gate=_dev_qt(R, g), up=_dev_qt(R, u))
    dout = torch.zeros(s * H, device="cuda")
    ctx.apply_single_expert(ds, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), s, k,
                            torch.from_numpy(x).cuda(), H, I, dout, activation=R.situ(4.0, lb))
    assert bits_equal(dout.cpu().numpy(), out)
    if kind == "mxfp4":
        gu = R.QT.mxfp4(np.concatenate([g.data, u.data]), np.concatenate([g.scale, u.scale]), 2 * I, H)
        fout = np.zeros(s * H, np.float32)
        ctx.apply_single_expert(R.Slot(5, rs.down, gate_up=gu), ids, w, s, k, x, H, I, fout,
                                activation=R.situ(4.0, lb))
        assert bits_equal(fout, out)


def test_apply_single_expert_activation_errors(ctx, orc):
    import rabbit_amd as R
    from rabbit_amd import abi
    H, I = 64, 32
    g, u, dn = orc.synth_mxfp4(I, H, 1), orc.synth_mxfp4(I, H, 2), orc.synth_mxfp4(H, I, 3)
    rs = R.Slot(0, _host_qt(R, dn), gate=_host_qt(R, g), up=_host_qt(R, u))
    ids, w = np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32)
    x, out = normal((1, H), 2), np.zeros(H, np.float32)
    for bad in (abi.RbtActivation(R.ACT_SITU, 0.0, 0.0, 0), abi.RbtActivation(R.ACT_SITU, 4.0, 0.0, 1),
                abi.RbtActivation(7, 1.0, 0.0, 0), abi.RbtActivation(R.ACT_SITU, float("nan"), 0.0, 0)):
        with pytest.raises(R.RbtError):
            ctx.apply_single_expert(rs, ids, w, 1, 1, x, H, I, out, activation=bad)
    with pytest.raises(R.RbtError):  # the int-activation entry point takes SiLU only
        ctx.apply_single_expert(rs, ids, w, 1, 1, x, H, I, out, activation=R.ACT_SITU)


def _latent_case(ctx, orc, layer, H, MH, I, E, k, seed, proj_kind, x_std, misalign=False):
    """Pool experts at (moe_hidden, moe_inter), a sigmoid router with a correction bias at full width
    (kimi_k3/moe.rs:232-262's layer shape), and the two projections. misalign: the device router
    starts 4 bytes past a 16-byte boundary."""
    import rabbit_amd as R
    import torch
    experts = {}
    for e in range(E):
        g = orc.synth_mxfp4(I, MH, seed + 3 * e)
        u = orc.synth_mxfp4(I, MH, seed + 3 * e + 1)
        dn = orc.synth_mxfp4(MH, I, seed + 3 * e + 2)
        experts[e] = orc.Slot(e, dn, gate=g, up=u)
        ctx.pool_put(layer, R.Slot(e, _host_qt(R, dn), gate=_host_qt(R, g), up=_host_qt(R, u)))
    router = normal((E, H), seed + 500, 0.05)
    bias = normal(E, seed + 501, 0.1)
    L = orc.MoeLayer(orc.FAMILY_GLM52, H, I, E, k, router, experts, router_bias=bias, norm_topk=False)
    t_router = torch.from_numpy(router).cuda()
    if misalign:
        buf = torch.zeros(E * H + 4, device="cuda")
        t_router = buf[1:1 + E * H]
        t_router.copy_(torch.from_numpy(router.ravel()).cuda())
    ctx.moe_layer_set(layer, R.FAMILY_GLM52, H, I, E, k, t_router,
                      router_bias=torch.from_numpy(bias).cuda(), norm_topk=False)
    if proj_kind == "f32":
        dq = orc.QT.f32(normal((MH, H), seed + 502, 0.05), MH, H)
        uq = orc.QT.f32(normal((H, MH), seed + 503, 0.05), H, MH)
    elif proj_kind == "i4g":
        dq, uq = orc.synth_i4g(MH, H, 32, seed + 502), orc.synth_i4g(H, MH, 32, seed + 503)
    else:
        dq, uq = orc.synth_mxfp4(MH, H, seed + 502), orc.synth_mxfp4(H, MH, seed + 503)
    torch.cuda.synchronize()
    return L, dq, uq, x_std


def _run_latent(ctx, R, layer, L, dq, uq, x, S, MH, norm, act_o, act_r):
    import torch
    H, k = L.hidden, L.topk
    exp, eids, ew = L.latent(x, S, MH, dq, uq, norm=norm, eps=1e-5, act=act_o)
    out = torch.empty(S * H, device="cuda")
    ids = torch.empty(S * k, dtype=torch.int32, device="cuda")
    w = torch.empty(S * k, device="cuda")
    ctx.latent_moe(layer, MH, _dev_qt(R, dq), _dev_qt(R, uq), torch.from_numpy(x).cuda(), S, out,
                   norm=None if norm is None else torch.from_numpy(norm).cuda(), eps=1e-5, activation=act_r,
                   ids_out=ids, w_out=w)
    assert np.array_equal(ids.cpu().numpy().reshape(S, k), eids)
    assert rel_l2(w.cpu().numpy().reshape(S, k), ew) < RTOL
    got = out.cpu().numpy().reshape(S, H)
    assert rel_l2(got, exp) < RTOL
    return got


# f32 projections take the separate norm kernel; MXFP4 and grouped-int4 ones the norm inside the up
# projection's GEMV
@pytest.mark.parametrize("proj_kind", ["f32", "mxfp4", "i4g"])
@pytest.mark.parametrize("S", [1, 3])
def test_latent_moe_matches_oracle(ctx, orc, proj_kind, S):
    import rabbit_amd as R
    H, MH, I, E, k = 256, 128, 64, 16, 4
    layer = 40 + {"f32": 0, "mxfp4": 2, "i4g": 4}[proj_kind] + (S == 3)
    L, dq, uq, _ = _latent_case(ctx, orc, layer, H, MH, I, E, k, 900 + layer, proj_kind, 1.0)
    x = normal((S, H), layer, 1.0)
    norm = np.abs(normal(MH, layer + 1, 1.0)) + np.float32(0.5)
    plain = _run_latent(ctx, R, layer, L, dq, uq, x, S, MH, None, None, None)
    normed = _run_latent(ctx, R, layer, L, dq, uq, x, S, MH, norm, None, None)
    assert rel_l2(plain, normed) > 1e-2  # the norm is applied (to the summed rows)
    situ = _run_latent(ctx, R, layer, L, dq, uq, x, S, MH, norm, orc.situ(4.0, 25.0), R.situ(4.0, 25.0))
    assert rel_l2(situ, normed) > 1e-3


# moe_hidden 6144 and 8192: the norm inside the up projection at its widest variants (each wave
# holds 3 or 4 KB-blocks of the summed row per lane beside the weight fragments)
@pytest.mark.parametrize("proj_kind", ["mxfp4", "i4g"])
@pytest.mark.parametrize("MH", [6144, 8192])
@pytest.mark.parametrize("S", [1, 3])
def test_latent_moe_wide_norm(ctx, orc, proj_kind, MH, S):
    import rabbit_amd as R
    H, I, E, k = 512, 64, 16, 4
    layer = 70 + (MH == 8192) * 4 + (proj_kind == "i4g") * 2 + (S == 3)
    L, dq, uq, _ = _latent_case(ctx, orc, layer, H, MH, I, E, k, 8000 + layer, proj_kind, 1.0)
    x = normal((S, H), layer, 1.0)
    norm = np.abs(normal(MH, layer + 1, 1.0)) + np.float32(0.5)
    plain = _run_latent(ctx, R, layer, L, dq, uq, x, S, MH, None, None, None)
    normed = _run_latent(ctx, R, layer, L, dq, uq, x, S, MH, norm, orc.situ(4.0, 25.0), R.situ(4.0, 25.0))
    assert rel_l2(plain, normed) > 1e-2


@pytest.mark.parametrize("misalign", [False, True])
def test_latent_moe_batch_exact_logits(ctx, orc, misalign):
    # 64 tokens: the router's logits are the reference's sequential folds themselves; a router that
    # is not 16-byte aligned takes the certified kernel instead, with the same ids
    import rabbit_amd as R
    H, MH, I, E, k, S = 256, 128, 64, 16, 4, 64
    layer = 60 + int(misalign)
    L, dq, uq, _ = _latent_case(ctx, orc, layer, H, MH, I, E, k, 6000 + layer, "mxfp4", 1.0, misalign=misalign)
    x = normal((S, H), layer, 1.0)
    norm = np.abs(normal(MH, layer + 1, 1.0)) + np.float32(0.5)
    _run_latent(ctx, R, layer, L, dq, uq, x, S, MH, norm, orc.situ(4.0, 25.0), R.situ(4.0, 25.0))


def test_latent_moe_k3_dims(ctx, orc):
    # Kimi K3's widths: hidden 7168, routed experts at moe_hidden 3584 with moe_inter 3072, top-8,
    # Situ(beta 4, linear_beta 25) and the routed-expert norm; 32 resident experts, 4 tokens (at
    # this shape about one token in four needs exact logit folds in the selection)
    import rabbit_amd as R
    H, MH, I, E, k, S = 7168, 3584, 3072, 32, 8, 4
    L, dq, uq, _ = _latent_case(ctx, orc, 50, H, MH, I, E, k, 7000, "mxfp4", 0.05)
    x = normal((S, H), 51, 0.05)
    norm = np.abs(normal(MH, 52, 0.2)) + np.float32(0.5)
    _run_latent(ctx, R, 50, L, dq, uq, x, S, MH, norm, orc.situ(4.0, 25.0), R.situ(4.0, 25.0))


@pytest.mark.parametrize("proj_kind", ["mxfp4", "i4g"])
def test_latent_moe_k3_dims_one_token(ctx, orc, proj_kind):
    # one token per call at K3's widths: the latent down projection streams inside the selection's
    # launch (workgroup 0 selects, the others project); six tokens, each its own call
    import rabbit_amd as R
    H, MH, I, E, k = 7168, 3584, 3072, 32, 8
    layer = 52 + (proj_kind == "i4g")
    L, dq, uq, _ = _latent_case(ctx, orc, layer, H, MH, I, E, k, 7100 + layer, proj_kind, 0.05)
    norm = np.abs(normal(MH, 53, 0.2)) + np.float32(0.5)
    for t in range(6):
        x = normal((1, H), 600 + t, 0.05)
        _run_latent(ctx, R, layer, L, dq, uq, x, 1, MH, norm, orc.situ(4.0, 25.0), R.situ(4.0, 25.0))


@pytest.mark.parametrize("k,tied", [(8, False), (2, True)])
def test_latent_moe_k3_folded_boundary_winner(ctx, orc, k, tied):
    # one token at K3's widths whose last top-k place only the exact folds decide (no correction
    # bias): helpers.boundary_router (two experts), the winner from the first undecided gate/up slot;
    # or at top-2 helpers.tied_boundary_router (five experts): k + 4 = 6 routed pairs stream, three
    # times top-k, each with its h row. The down GEMV and the combine take the winner's row by rank.
    import rabbit_amd as R
    import torch
    from helpers import boundary_router, tied_boundary_router
    H, MH, I, E, layer = 7168, 3584, 3072, 32, 54 + 10 * tied
    L, dq, uq, _ = _latent_case(ctx, orc, layer, H, MH, I, E, k, 7300, "i4g", 0.05)
    x = normal((1, H), 610, 0.05)
    if tied:
        router, cands, _, _ = tied_boundary_router(E, H, k, x[0])
        b = cands[-1]
    else:
        router, a, b, _ = boundary_router(E, H, k, x[0])
    bias = np.zeros(E, np.float32)
    L = orc.MoeLayer(orc.FAMILY_GLM52, H, I, E, k, router, L.experts, router_bias=bias, norm_topk=False)
    t_router, t_bias = torch.from_numpy(router).cuda(), torch.from_numpy(bias).cuda()
    ctx.moe_layer_set(layer, R.FAMILY_GLM52, H, I, E, k, t_router, router_bias=t_bias, norm_topk=False)
    torch.cuda.synchronize()
    norm = np.abs(normal(MH, 55, 0.2)) + np.float32(0.5)
    ctx.profile_read(reset=True)
    got = _run_latent(ctx, R, layer, L, dq, uq, x, 1, MH, norm, orc.situ(4.0, 25.0), R.situ(4.0, 25.0))
    assert ctx.profile_read(reset=True)["ambiguous"], "the router decision did not need exact folds"
    assert np.all(np.isfinite(got))
    ids = torch.empty(k, dtype=torch.int32, device="cuda")
    ctx.latent_moe(layer, MH, _dev_qt(R, dq), _dev_qt(R, uq), torch.from_numpy(x).cuda(), 1,
                   torch.empty(H, device="cuda"), norm=torch.from_numpy(norm).cuda(), eps=1e-5,
                   activation=R.situ(4.0, 25.0), ids_out=ids)
    assert b in list(ids.cpu().numpy())


def test_latent_moe_k3_graph_replays(ctx, orc):
    # one token at K3's widths (the key-record router, the selection in the gate/up launch) captured
    # in a HIP graph as the benchmark replays it, and replayed with other inputs, eager calls between
    # the replays: every replay equals the eager result
    import rabbit_amd as R
    import torch
    from helpers import HipGraph
    H, MH, I, E, k = 7168, 3584, 3072, 32, 8
    layer = 54
    L, dq, uq, _ = _latent_case(ctx, orc, layer, H, MH, I, E, k, 7300, "i4g", 0.05)
    norm = torch.from_numpy(np.abs(normal(MH, 55, 0.2)) + np.float32(0.5)).cuda()
    dqd, uqd, act = _dev_qt(R, dq), _dev_qt(R, uq), R.situ(4.0, 25.0)
    xs = [torch.from_numpy(normal((1, H), 700 + t, 0.05)).cuda() for t in range(3)]

    def call(x, out, sync=True):
        ctx.latent_moe(layer, MH, dqd, uqd, x, 1, out, norm=norm, eps=1e-5, activation=act, sync=sync)

    ref = []
    for t in range(3):
        o = torch.empty(H, device="cuda")
        call(xs[t], o)
        ref.append(o.cpu().numpy())
    xin = xs[0].clone()
    gout = torch.empty(H, device="cuda")
    call(xin, gout)  # scratch sized before the capture
    torch.cuda.synchronize()
    g = HipGraph(ctx.stream)
    g.begin()
    call(xin, gout, sync=False)
    g.end()
    try:
        for rep in range(6):
            t = rep % 3
            xin.copy_(xs[t])
            torch.cuda.synchronize()
            g.launch()
            ctx.sync()
            assert np.array_equal(gout.cpu().numpy(), ref[t]), rep
            u = (t + 1) % 3
            o = torch.empty(H, device="cuda")
            call(xs[u], o)
            assert np.array_equal(o.cpu().numpy(), ref[u]), rep
    finally:
        g.destroy()


def test_latent_moe_identity_projections_equal_routed_forward(ctx, orc):
    # moe_hidden == hidden with identity projections: the latent MoE is the layer's routed forward
    import rabbit_amd as R
    import torch
    H, I, E, k, S = 256, 64, 16, 4, 3
    L, _, _, _ = _latent_case(ctx, orc, 55, H, H, I, E, k, 5500, "f32", 1.0)
    eye = orc.QT.f32(np.eye(H, dtype=np.float32).ravel(), H, H)
    x = normal((S, H), 56, 1.0)
    lat = _run_latent(ctx, R, 55, L, eye, eye, x, S, H, None, None, None)
    out = torch.empty(S * H, device="cuda")
    ctx.moe_forward(55, torch.from_numpy(x).cuda(), S, out)
    assert rel_l2(out.cpu().numpy().reshape(S, H), lat) < RTOL


def test_latent_moe_errors(ctx, orc):
    import rabbit_amd as R
    import torch
    H, MH, I, E, k = 256, 128, 64, 16, 4
    L, dq, uq, _ = _latent_case(ctx, orc, 57, H, MH, I, E, k, 5700, "f32", 1.0)
    x = torch.from_numpy(normal((1, H), 58)).cuda()
    out = torch.empty(H, device="cuda")
    with pytest.raises(R.RbtError):  # projections transposed
        ctx.latent_moe(57, MH, _dev_qt(R, uq), _dev_qt(R, dq), x, 1, out)
    with pytest.raises(R.RbtError):  # experts are not shaped for this moe_hidden
        wrong = orc.QT.f32(np.zeros(64 * H, np.float32), 64, H)
        ctx.latent_moe(57, 64, _dev_qt(R, wrong), _dev_qt(R, orc.QT.f32(np.zeros(H * 64, np.float32), H, 64)), x, 1,
                       out)
    with pytest.raises(R.RbtError):  # no such layer
        ctx.latent_moe(99, MH, _dev_qt(R, dq), _dev_qt(R, uq), x, 1, out)
