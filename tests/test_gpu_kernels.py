"""GPU parity: the HIP kernels through the C ABI against the CPU oracle on the same seeded inputs.

Bars: dequantized MXFP4 / int4 weights and top-k expert ids bit-exact; fp32-accumulated outputs
within 1e-5 relative L2 (RTOL below).
"""
import numpy as np
import pytest

from helpers import bits_equal, normal, rel_l2, xorshift_vec

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _np(t):
    return t.cpu().numpy()


def test_version_and_context(ctx):
    assert b"gfx950" in ctx.lib.rbt_version()


def test_synth_device_matches_host(ctx, orc):
    import torch
    rows, cols = 64, 416
    d = torch.empty(rows * cols // 2, dtype=torch.uint8, device="cuda")
    s = torch.empty(rows * cols // 32, dtype=torch.uint8, device="cuda")
    ctx.synth_mxfp4(d.data_ptr(), s.data_ptr(), rows, cols, 77, 119, 123)
    ctx.sync()
    h = orc.synth_mxfp4(rows, cols, 77, 119, 123)
    assert np.array_equal(_np(d), h.data) and np.array_equal(_np(s), h.scale)
    gs = 32
    d2 = torch.empty(rows * cols // 2, dtype=torch.uint8, device="cuda")
    s2 = torch.empty(rows * cols // gs, dtype=torch.float32, device="cuda")
    ctx.synth_i4g(d2.data_ptr(), s2.data_ptr(), rows, cols, gs, 78, 0.005, 0.02)
    ctx.sync()
    h2 = orc.synth_i4g(rows, cols, gs, 78, 0.005, 0.02)
    assert np.array_equal(_np(d2), h2.data) and bits_equal(_np(s2), h2.scale)


# ---- dequant: bit-exact ------------------------------------------------------------------------
def test_dequant_mxfp4_bit_exact_every_byte_every_scale(ctx, orc):
    import rabbit_amd as R
    rows, cols = 256, 512  # row r: all 256 data bytes, every block scaled by byte r
    data = np.tile(np.arange(256, dtype=np.uint8), rows)
    scale = np.repeat(np.arange(256, dtype=np.uint8), cols // 32)
    hq = orc.QT.mxfp4(data, scale, rows, cols)
    exp = hq.dense()
    got = ctx.dequant_rows(R.QT.mxfp4(data, scale, rows, cols), 0, rows).reshape(rows, cols)
    assert bits_equal(got, exp)
    got_d = _np(ctx.dequant_rows(R.QT.mxfp4(_t(data), _t(scale), rows, cols), 0, rows)).reshape(rows, cols)
    assert bits_equal(got_d, exp)


def test_dequant_i4g_bit_exact(ctx, orc):
    import rabbit_amd as R
    rows, cols, gs = 33, 70, 16
    hq = orc.synth_i4g(rows, cols, gs, seed=3)
    got = ctx.dequant_rows(R.QT.i4g(hq.data, hq.scale, rows, cols, gs), 5, 20).reshape(20, cols)
    assert bits_equal(got, hq.dense()[5:25])


# ---- the fp4 conversion inside the decode GEMV: one-hot activations read back W's columns --------
@pytest.mark.parametrize("scale_bytes", [(119, 123), (100, 140), (1, 8), (240, 252)])
def test_decode_gemv_reads_exact_weights(ctx, orc, scale_bytes):
    import torch
    rows, cols = 64, 8192
    hq = orc.synth_mxfp4(rows, cols, seed=11, exp_lo=scale_bytes[0], exp_hi=scale_bytes[1])
    dense = hq.dense()
    probe = [0, 1, 2, 31, 32, 33, 4095, 8191]
    x = np.zeros((len(probe), cols), np.float32)
    for s, k in enumerate(probe):
        x[s, k] = 1.0
    y = torch.empty(len(probe) * rows, dtype=torch.float32, device="cuda")
    ctx.matmul_mxfp4(y, _t(x), _t(hq.data), _t(hq.scale), len(probe), cols, rows)
    got = _np(y).reshape(len(probe), rows)
    for s, k in enumerate(probe):
        assert np.array_equal(got[s], dense[:, k]), (scale_bytes, k)


def test_decode_gemv_scale_byte_zero(ctx, orc):
    # E8M0 byte 0 is the subnormal 2^-127 (quant.rs:391-396); products stay exact with x = 2^100.
    import torch
    rows, cols = 16, 1024
    hq = orc.synth_mxfp4(rows, cols, seed=12, exp_lo=0, exp_hi=0)
    x = np.zeros((1, cols), np.float32)
    x[0, 5] = 2.0 ** 100
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul_mxfp4(y, _t(x), _t(hq.data), _t(hq.scale), 1, cols, rows)
    assert np.array_equal(_np(y), (hq.dense()[:, 5].astype(np.float64) * 2.0 ** 100).astype(np.float32))


# ---- one token on the matrix cores (k_xgemv1): exact weights, scale byte 0, benchmark shapes -----
@pytest.mark.parametrize("rows,cols", [(64, 8192), (3072, 3584), (8192, 2048)])
def test_one_token_matmul_reads_exact_weights(ctx, orc, rows, cols):
    """One token per call (the single-token matrix-core path): a one-hot activation reads back one
    weight column bit for bit (the E2M1 x E8M0 decode and the three-part split of x are exact)."""
    import torch
    hq = orc.synth_mxfp4(rows, cols, seed=13 + rows, exp_lo=100, exp_hi=140)
    dense = hq.dense()
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    for k in (0, 1, 31, 32, 511, 512, cols - 1):
        x = np.zeros((1, cols), np.float32)
        x[0, k] = 1.0
        ctx.matmul_mxfp4(y, _t(x), _t(hq.data), _t(hq.scale), 1, cols, rows)
        assert np.array_equal(_np(y), dense[:, k]), k


def test_one_token_matmul_scale_byte_zero(ctx, orc):
    # E8M0 byte 0 is the subnormal 2^-127 (quant.rs:391-396) on the single-token path too
    import torch
    rows, cols = 64, 2048
    hq = orc.synth_mxfp4(rows, cols, seed=14, exp_lo=0, exp_hi=0)
    x = np.zeros((1, cols), np.float32)
    x[0, 5] = 2.0 ** 100
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul_mxfp4(y, _t(x), _t(hq.data), _t(hq.scale), 1, cols, rows)
    assert np.array_equal(_np(y), (hq.dense()[:, 5].astype(np.float64) * 2.0 ** 100).astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(3072, 3584), (4096, 4096), (2048, 8192), (8192, 2048), (2048, 7168),
                                       (7168, 2048)])
def test_one_token_matmul_parity(ctx, orc, rows, cols):
    """matmul_mxfp4 for one token at the reference's micro-benchmark shapes (benches/kernels.rs:
    209-240, 310-343) and C0's matrices: within 1e-5 of the scalar tier."""
    import torch
    hq = orc.synth_mxfp4(rows, cols, seed=rows * 3 + cols)
    x = normal((1, cols), seed=rows)
    exp = orc.matmul_mxfp4_scalar(x, hq.data, hq.scale, 1, cols, rows)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    ctx.matmul_mxfp4(y, _t(x), _t(hq.data), _t(hq.scale), 1, cols, rows)
    assert rel_l2(_np(y), exp) < RTOL


# ---- matmul parity ------------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols,s", [(2048, 8192, 1), (8192, 2048, 1), (2048, 6144, 1), (7168, 2048, 1),
                                         (2048, 7168, 1), (300, 8192, 3), (64, 96, 2)])
def test_matmul_mxfp4_parity(ctx, orc, rows, cols, s):
    import torch
    hq = orc.synth_mxfp4(rows, cols, seed=rows + cols + s)
    x = normal((s, cols), seed=s)
    exp = orc.matmul_mxfp4_scalar(x, hq.data, hq.scale, s, cols, rows)
    y = torch.empty(s * rows, dtype=torch.float32, device="cuda")
    ctx.matmul_mxfp4(y, _t(x), _t(hq.data), _t(hq.scale), s, cols, rows)
    assert rel_l2(_np(y), exp) < RTOL
    yh = np.empty(s * rows, np.float32)
    ctx.matmul_mxfp4(yh, x, hq.data, hq.scale, s, cols, rows)
    assert bits_equal(yh, _np(y))


@pytest.mark.parametrize("cols", [1, 7, 16, 17, 32, 33, 65])
def test_matmul_mxfp4_tails(ctx, orc, cols):
    rows = 3
    hq = orc.synth_mxfp4(rows, cols, seed=cols * 3 + 9, exp_lo=120, exp_hi=134)
    for s in (1, 2):
        x = xorshift_vec(s * cols, cols * 7 + 10)
        exp = orc.matmul_mxfp4_scalar(x, hq.data, hq.scale, s, cols, rows)
        y = np.empty(s * rows, np.float32)
        ctx.matmul_mxfp4(y, x, hq.data, hq.scale, s, cols, rows)
        assert np.max(np.abs(y - exp)) < 1e-4 and rel_l2(y, exp) < RTOL


@pytest.mark.parametrize("rows,cols,gs,s", [(2048, 6144, 32, 1), (6144, 2048, 32, 1), (37, 70, 16, 2),
                                            (5, 33, 32, 1), (64, 256, 64, 3)])
def test_matmul_i4g_parity(ctx, orc, rows, cols, gs, s):
    hq = orc.synth_i4g(rows, cols, gs, seed=rows + cols)
    x = normal((s, cols), seed=5)
    exp = orc.matmul_i4_grouped(x, hq.data, hq.scale, gs, s, cols, rows)
    y = np.empty(s * rows, np.float32)
    ctx.matmul_i4_grouped(y, x, hq.data, hq.scale, gs, s, cols, rows)
    assert rel_l2(y, exp) < RTOL


def test_matmul_f32_parity(ctx, orc):
    s, i, o = 3, 8192, 512
    x = normal((s, i), 1)
    w = normal((o, i), 2, 0.02)
    exp = orc.matmul(x, w, s, i, o)
    y = np.empty(s * o, np.float32)
    ctx.matmul(y, x, w, s, i, o)
    assert rel_l2(y, exp) < RTOL
    k = {"x": [1.0, 2.0, 3.0, -1.0, 0.5, 2.0], "w": [1.0, 0.0, 0.0, 0.0, 1.0, 1.0]}
    y = np.empty(4, np.float32)
    ctx.matmul(y, np.array(k["x"], np.float32), np.array(k["w"], np.float32), 2, 3, 2)
    assert list(y) == [1.0, 5.0, -1.0, 2.5]  # kernels.rs:1323-1331


def test_mxfp4_two_block_kat_gpu(ctx):
    cols = 40
    data = np.array([4 | (4 << 4)] * 16 + [(7 | 8) | ((7 | 8) << 4)] * 4, np.uint8)
    y = np.empty(1, np.float32)
    ctx.matmul_mxfp4(y, np.ones(cols, np.float32), data, np.array([127, 130], np.uint8), 1, cols, 1)
    assert y[0] == -320.0  # kernels.rs:1388-1406


# ---- routers -------------------------------------------------------------------------------------
def test_route_softmax_kats_gpu(ctx, orc):
    import json
    import os
    kats = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kats.json")))
    from golden.make_golden import lcg_logits
    for c in kats["route_hf"]["cases"]:
        ids = np.empty(10, np.int32)
        w = np.empty(10, np.float32)
        ctx.route_softmax_topk(lcg_logits(512, c["seed"]), 1, 512, 10, ids, w)
        assert list(ids) == c["ids"] and np.max(np.abs(w - np.array(c["weights"]))) < 1e-6
    for c in kats["route_ties"]["cases"] + [dict(kats["route_select"])]:
        n = len(c["logits"])
        ids = np.empty(c["k"], np.int32)
        w = np.empty(c["k"], np.float32)
        ctx.route_softmax_topk(np.array(c["logits"], np.float32), 1, n, c["k"], ids, w)
        assert list(ids) == c["ids"]
    ids = np.empty(3, np.int32)
    w = np.empty(3, np.float32)
    ctx.route_softmax_topk(np.array([3.0, 1.0, 2.0], np.float32), 1, 3, 10, ids, w)
    assert list(ids) == [0, 2, 1] and abs(w.sum() - 1) < 1e-6


def test_route_random_matches_oracle(ctx, orc):
    s, n, k = 64, 512, 10
    logits = normal((s, n), 9, 2.0)
    logits[:, 100] = logits[:, 101]  # exact ties resolve to the lower id
    ids = np.empty(s * k, np.int32)
    w = np.empty(s * k, np.float32)
    ctx.route_softmax_topk(logits, s, n, k, ids, w)
    for t in range(s):
        ri, rw = orc.route_softmax(logits[t], k)
        assert list(ids[t * k:(t + 1) * k]) == list(ri)
        assert np.max(np.abs(w[t * k:(t + 1) * k] - rw)) < 1e-6
    bias = normal(n, 4, 0.01)
    ctx.route_sigmoid_topk(logits, bias, s, n, 8, True, 2.5, ids[:s * 8], w[:s * 8])
    for t in range(s):
        ri, rw = orc.route_sigmoid(logits[t], 8, bias=bias, norm_topk=True, routed_scale=2.5)
        assert list(ids[t * 8:(t + 1) * 8]) == list(ri)
        assert np.max(np.abs(w[t * 8:(t + 1) * 8] - rw)) < 1e-6
    # grouped top-k (glm52/moe.rs:214-229)
    ctx.route_sigmoid_topk(logits, None, s, n, 8, False, 1.0, ids[:s * 8], w[:s * 8], n_group=8, topk_group=3)
    for t in range(s):
        ri, _ = orc.route_sigmoid(logits[t], 8, norm_topk=False, n_group=8, topk_group=3)
        assert list(ids[t * 8:(t + 1) * 8]) == list(ri)


# ---- experts -------------------------------------------------------------------------------------
def test_apply_single_expert_c0(ctx, orc):
    """Config 0: one MXFP4 SwiGLU expert (gate/up [2048, 8192], down [8192, 2048]), one token."""
    import rabbit_amd as R
    H, I = 8192, 2048
    g, u, dn = orc.synth_mxfp4(I, H, 1), orc.synth_mxfp4(I, H, 2), orc.synth_mxfp4(H, I, 3)
    slot = orc.Slot(0, dn, gate=g, up=u)
    x = normal((1, H), 7)
    ids = np.zeros((1, 1), np.int32)
    w = np.ones((1, 1), np.float32)
    exp = orc.apply_single_expert(slot, ids, w, x, H, I, np.zeros(H, np.float32))
    rs = R.Slot(0, R.QT.mxfp4(dn.data, dn.scale, H, I), gate=R.QT.mxfp4(g.data, g.scale, I, H),
                up=R.QT.mxfp4(u.data, u.scale, I, H))
    out = np.zeros(H, np.float32)
    ctx.apply_single_expert(rs, ids, w, 1, 1, x, H, I, out)
    assert rel_l2(out, exp) < RTOL
    # fused gate_up == separate, bit-exact (glm52/moe.rs:592-626)
    fused = R.Slot(0, rs.down, gate_up=R.QT.mxfp4(np.concatenate([g.data, u.data]),
                                                  np.concatenate([g.scale, u.scale]), 2 * I, H))
    out2 = np.zeros(H, np.float32)
    ctx.apply_single_expert(fused, ids, w, 1, 1, x, H, I, out2)
    assert bits_equal(out, out2)


@pytest.mark.parametrize("H", [8192, 7168])
def test_apply_single_expert_one_token_routing(ctx, orc, H):
    """One token, k = 3 (the single-token matrix-core path): the expert's first matching slot gives
    the weight (glm52/moe.rs:465-470), out accumulates onto what it held; a token that did not pick
    the expert leaves out untouched; Situ runs on this path too."""
    import rabbit_amd as R
    I = 2048
    g, u, dn = orc.synth_mxfp4(I, H, 21), orc.synth_mxfp4(I, H, 22), orc.synth_mxfp4(H, I, 23)
    slot = orc.Slot(7, dn, gate=g, up=u)
    rs = R.Slot(7, R.QT.mxfp4(dn.data, dn.scale, H, I), gate=R.QT.mxfp4(g.data, g.scale, I, H),
                up=R.QT.mxfp4(u.data, u.scale, I, H))
    x = normal((1, H), 24)
    base = normal((1, H), 25).ravel()
    ids = np.array([[3, 7, 7]], np.int32)
    w = np.array([[0.5, -0.75, 2.0]], np.float32)
    exp = orc.apply_single_expert(slot, ids, w, x, H, I, base.copy())
    out = base.copy()
    ctx.apply_single_expert(rs, ids, w, 1, 3, x, H, I, out)
    assert rel_l2(out - base, exp - base) < RTOL
    miss = base.copy()
    ctx.apply_single_expert(rs, np.array([[1, 2, 3]], np.int32), w, 1, 3, x, H, I, miss)
    assert np.array_equal(miss, base)
    xs = normal((1, H), 26, 0.5)
    exp_s = orc.apply_single_expert(slot, ids, w, xs, H, I, np.zeros(H, np.float32), act=orc.situ(4.0, 25.0))
    out_s = np.zeros(H, np.float32)
    ctx.apply_single_expert(rs, ids, w, 1, 3, xs, H, I, out_s, activation=R.situ(4.0, 25.0))
    assert rel_l2(out_s, exp_s) < RTOL


def test_apply_single_expert_multi_token_accumulates(ctx, orc):
    import rabbit_amd as R
    H, I, s, k = 512, 256, 5, 3
    g, u, dn = orc.synth_mxfp4(I, H, 4), orc.synth_mxfp4(I, H, 5), orc.synth_mxfp4(H, I, 6)
    slot = orc.Slot(7, dn, gate=g, up=u)
    x = normal((s, H), 8)
    ids = np.array([[7, 1, 2], [3, 4, 5], [1, 7, 0], [7, 9, 8], [2, 3, 7]], np.int32)
    w = normal((s, k), 9)
    base = normal((s, H), 10)
    exp = orc.apply_single_expert(slot, ids, w, x, H, I, base.copy().ravel())
    rs = R.Slot(7, R.QT.mxfp4(dn.data, dn.scale, H, I), gate=R.QT.mxfp4(g.data, g.scale, I, H),
                up=R.QT.mxfp4(u.data, u.scale, I, H))
    out = base.copy().ravel()
    ctx.apply_single_expert(rs, ids, w, s, k, x, H, I, out)
    assert rel_l2(out, exp) < RTOL
    assert np.array_equal(out.reshape(s, H)[1], base[1])  # token 1 did not pick expert 7


def test_apply_single_expert_i4g_odd_shape(ctx, orc):
    import rabbit_amd as R
    H, I, gs = 70, 24, 16
    g, u, dn = orc.synth_i4g(I, H, gs, 1), orc.synth_i4g(I, H, gs, 2), orc.synth_i4g(H, I, gs, 3)
    slot = orc.Slot(0, dn, gate=g, up=u)
    x = normal((2, H), 1)
    ids = np.zeros((2, 1), np.int32)
    w = np.array([[0.7], [-1.2]], np.float32)
    exp = orc.apply_single_expert(slot, ids, w, x, H, I, np.zeros(2 * H, np.float32))
    rs = R.Slot(0, R.QT.i4g(dn.data, dn.scale, H, I, gs), gate=R.QT.i4g(g.data, g.scale, I, H, gs),
                up=R.QT.i4g(u.data, u.scale, I, H, gs))
    out = np.zeros(2 * H, np.float32)
    ctx.apply_single_expert(rs, ids, w, 2, 1, x, H, I, out)
    assert rel_l2(out, exp) < RTOL
