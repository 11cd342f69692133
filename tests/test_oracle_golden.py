"""Pins the CPU oracle: the reference's own known-answer tests (tests/golden/kats.json), closed forms,
and brute force on small inputs. Each check is chosen so that a plausible restatement mistake (a
dropped term, a wrong sign or index, a fused multiply-add, a transposed operand) fails it."""
import json
import math
import os

import numpy as np
import pytest

from helpers import bits_equal, rel_l2, xorshift_vec

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kats.json")))


def f32(v):
    return np.float32(v)


# ---- quant.rs ---------------------------------------------------------------------------------
def test_e2m1_table_kat(orc):
    k = KATS["e2m1_table"]
    got = np.array([orc.e2m1_decode(c) for c in k["codes"]], np.float32)
    assert bits_equal(got, np.array(k["values"], np.float32))  # includes -0.0 for code 8


def test_e8m0_points_and_exhaustive_powers_of_two(orc):
    k = KATS["e8m0_points"]
    for b, v in zip(k["bytes"], k["values"]):
        assert orc.e8m0_decode(b) == v
    # quant.rs:895-905: every byte 0..254 equals 2^(b-127) exactly (byte 0 is the subnormal 2^-127)
    for b in range(255):
        assert orc.e8m0_decode(b) == math.ldexp(1.0, b - 127), b
    assert orc.e8m0_decode_bits(255) == 0x7F800000  # quant.rs:391-396: +inf bits, not NaN
    assert orc.e8m0_decode_bits(0) == 1 << 22


def test_row_f32_disk_bytes_kat(orc):
    k = KATS["disk_bytes"]
    q = orc.QT.mxfp4(np.array(k["data"], np.uint8), np.array(k["scale"], np.uint8), 1, k["cols"])
    assert bits_equal(q.row_f32(0), np.array(k["row0"], np.float32))


def test_row_f32_mxfp4_closed_form_every_byte_and_scale(orc):
    # Every data byte with every scale byte: w = e2m1(n) * 2^(b-127) exactly (quant.rs:325-339).
    mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    data = np.arange(256, dtype=np.uint8)  # one row of 512 elements = 16 blocks
    for sb in list(range(0, 256, 7)) + [0, 1, 254, 255]:
        scale = np.full(16, sb, np.uint8)
        got = orc.QT.mxfp4(data, scale, 1, 512).row_f32(0)
        sc = math.ldexp(1.0, sb - 127) if sb < 255 else math.inf
        exp = []
        for byte in range(256):
            for nib in (byte & 0xF, byte >> 4):
                m = mags[nib & 7]
                v = np.float32(m) * np.float32(sc) if not (m == 0.0 and sc == math.inf) else np.float32(np.nan)
                exp.append(-v if nib & 8 else v)
        assert bits_equal(got, np.array(exp, np.float32)), sb


def test_row_f32_i4g_closed_form(orc):
    rows, cols, gs = 3, 37, 8  # partial trailing group (quant.rs:606-623 fixture shape)
    rng = np.random.default_rng(0)
    nib = rng.integers(0, 16, (rows, cols))
    data = np.zeros((rows, (cols + 1) // 2), np.uint8)
    for r in range(rows):
        for k in range(cols):
            data[r, k // 2] |= nib[r, k] << (4 * (k % 2))
    ng = (cols + gs - 1) // gs
    scale = rng.uniform(0.005, 0.02, (rows, ng)).astype(np.float32)
    q = orc.QT.i4g(data, scale, rows, cols, gs)
    for r in range(rows):
        exp = np.array([np.float32(nib[r, k] - 8) * scale[r, k // gs] for k in range(cols)], np.float32)
        assert bits_equal(q.row_f32(r), exp)


def test_resident_bytes(orc):
    # quant.rs:1011-1017 (resident_bytes_matches_format) plus the MXFP4/grouped formulas
    assert orc.QT.mxfp4(np.zeros(10 * 50, np.uint8), np.zeros(10 * 4, np.uint8), 10, 100).resident_bytes() == \
        10 * 50 + 10 * 4
    assert orc.QT.i4g(np.zeros(10 * 50, np.uint8), np.zeros(10 * 4, np.float32), 10, 100, 25).resident_bytes() == \
        10 * 50 + 10 * 4 * 4


# ---- kernels.rs --------------------------------------------------------------------------------
def test_matmul_kat(orc):
    k = KATS["matmul"]
    y = orc.matmul(np.array(k["x"], np.float32), np.array(k["w"], np.float32), k["s"], k["i"], k["o"])
    assert list(y) == k["y"]


def seq_dot_f32(x, w):
    """Left-to-right fold of rounded f32 products, one rounding per operation (pure Python)."""
    a = np.float32(-0.0)
    for xv, wv in zip(x.astype(np.float32), w.astype(np.float32)):
        a = np.float32(a + np.float32(xv * wv))
    return a


def test_matmul_sequential_order_brute_force(orc):
    s, i, o = 2, 301, 5
    x = xorshift_vec(s * i, 7) * 3
    w = xorshift_vec(o * i, 8)
    y = orc.matmul(x, w, s, i, o).reshape(s, o)
    for si in range(s):
        for oi in range(o):
            assert y[si, oi] == seq_dot_f32(x[si * i:(si + 1) * i], w[oi * i:(oi + 1) * i])


def test_mxfp4_two_block_kat(orc):
    k = KATS["mxfp4_two_block"]
    args = (np.array(k["x"], np.float32), np.array(k["data"], np.uint8), np.array(k["block_scale"], np.uint8), 1,
            k["cols"], 1)
    assert list(orc.matmul_mxfp4_scalar(*args)) == k["y"]
    assert list(orc.matmul_mxfp4_tier(*args)) == k["y"]


def test_i4g_two_group_kat(orc):
    k = KATS["i4g_two_group"]
    y = orc.matmul_i4_grouped(np.array(k["x"], np.float32), np.array(k["q4"], np.uint8),
                              np.array(k["scale"], np.float32), k["gs"], 1, k["cols"], 1)
    assert list(y) == k["y"]


def test_mxfp4_scalar_brute_force_sequential(orc):
    # a += (x*e2m1)*e8m0, sequential, no FMA (kernels.rs:247-267); odd cols and a partial block
    rows, cols, s = 4, 77, 2
    q = orc.synth_mxfp4(rows, cols, seed=5, exp_lo=100, exp_hi=140)
    x = xorshift_vec(s * cols, 3)
    y = orc.matmul_mxfp4_scalar(x, q.data, q.scale, s, cols, rows).reshape(s, rows)
    dense = q.dense()
    for si in range(s):
        for r in range(rows):
            a = np.float32(0.0)
            for k in range(cols):
                e = dense[r, k]
                sc = np.float32(math.ldexp(1.0, int(q.scale[r * 3 + k // 32]) - 127))
                m = np.float32(e / sc)  # exact: e2m1 value
                a = np.float32(a + np.float32(np.float32(x[si * cols + k] * m) * sc))
            assert y[si, r] == a


def test_i4g_brute_force_sequential(orc):
    rows, cols, gs, s = 3, 70, 16, 2
    q = orc.synth_i4g(rows, cols, gs, seed=9)
    x = xorshift_vec(s * cols, 4)
    y = orc.matmul_i4_grouped(x, q.data, q.scale, gs, s, cols, rows).reshape(s, rows)
    ng = (cols + gs - 1) // gs
    for si in range(s):
        for r in range(rows):
            a = np.float32(0.0)
            for k in range(cols):
                byte = q.data[r * ((cols + 1) // 2) + k // 2]
                n = (byte >> (4 * (k % 2))) & 0xF
                a = np.float32(a + np.float32(np.float32(x[si * cols + k] * np.float32(int(n) - 8)) *
                                              q.scale[r * ng + k // gs]))
            assert y[si, r] == a


def test_matmul_qt_mxfp4_matches_dequant_dot(orc):
    # kernels.rs:1570-1596: within 1e-3 of row_f32 dotted sequentially
    rows, cols, s = 5, 96, 2
    q = orc.synth_mxfp4(rows, cols, seed=31)
    x = xorshift_vec(s * cols, 32)
    dense = q.dense().astype(np.float64)
    exp = (x.reshape(s, cols).astype(np.float64) @ dense.T)
    for simd in (False, True):
        y = orc.matmul_qt(x, q, s, simd=simd).reshape(s, rows)
        assert np.max(np.abs(y - exp)) < 1e-3


@pytest.mark.parametrize("tier", ["avx2", "avx512"])
def test_simd_tiers_within_tolerance_of_scalar(orc, tier):
    k = KATS["tier_cols"]
    if tier == "avx512" and not orc.lib().orc_cpu_has_avx512():
        pytest.skip("no AVX-512F/BW")
    if tier == "avx2" and not orc.lib().orc_cpu_has_avx2():
        pytest.skip("no AVX2")
    for cols in k["cols"]:
        q = orc.synth_mxfp4(k["rows"], cols, seed=cols * 3 + 9, exp_lo=120, exp_hi=134)
        x = xorshift_vec(cols, cols * 7 + 10)
        ys = orc.matmul_mxfp4_scalar(x, q.data, q.scale, 1, cols, k["rows"])
        yt = orc.matmul_mxfp4_tier(x, q.data, q.scale, 1, cols, k["rows"], tier=tier)
        assert np.max(np.abs(ys - yt)) < k["tol"], cols


def test_simd_tier_large_rel_l2(orc):
    q = orc.synth_mxfp4(64, 8192, seed=1)
    x = np.random.default_rng(1).standard_normal(8192).astype(np.float32)
    ys = orc.matmul_mxfp4_scalar(x, q.data, q.scale, 1, 8192, 64)
    yt = orc.matmul_mxfp4_tier(x, q.data, q.scale, 1, 8192, 64)
    assert rel_l2(yt, ys) < 1e-5


# ---- routers -----------------------------------------------------------------------------------
def test_route_select_kat(orc):
    k = KATS["route_select"]
    ids, w = orc.route_softmax(np.array(k["logits"], np.float32), k["k"])
    assert list(ids) == k["ids"]
    assert w[0] > w[1] > w[2]


def test_route_ties_and_k_ge_n(orc):
    for c in KATS["route_ties"]["cases"]:
        ids, _ = orc.route_softmax(np.array(c["logits"], np.float32), c["k"])
        assert list(ids) == c["ids"]
    k = KATS["route_k_ge_n"]
    ids, w = orc.route_softmax(np.array(k["logits"], np.float32), k["k"])
    assert list(ids) == k["ids"] and abs(float(w.sum()) - 1.0) < 1e-6
    ids, w = orc.route_softmax(np.array(k["logits"], np.float32), 0)
    assert len(ids) == 0


def test_route_matches_hf_transcription(orc):
    from golden.make_golden import lcg_logits
    k = KATS["route_hf"]
    for c in k["cases"]:
        ids, w = orc.route_softmax(lcg_logits(k["n"], c["seed"]), k["k"])
        assert list(ids) == c["ids"]
        assert np.max(np.abs(w - np.array(c["weights"], np.float32))) < k["tol"]


def test_route_shift_invariance(orc):
    from golden.make_golden import lcg_logits
    l = lcg_logits(128, 11)
    a_ids, a_w = orc.route_softmax(l, 10)
    b_ids, b_w = orc.route_softmax((l + np.float32(17.5)).astype(np.float32), 10)
    assert list(a_ids) == list(b_ids) and np.max(np.abs(a_w - b_w)) < 1e-6


def test_glm_selection_uses_biased_score_weight_uses_plain_sigmoid(orc):
    k = KATS["glm_select_vs_weight"]
    logits = orc.matmul(np.array(k["x"], np.float32), np.array(k["router"], np.float32), 1, 2, 2)
    ids, w = orc.route_sigmoid(logits, k["k"], bias=np.array(k["bias"], np.float32), norm_topk=False)
    assert list(ids) == k["ids"] and abs(w[0] - k["weight"]) < k["tol"]


def test_glm_norm_topk_sums_to_routed_scale(orc):
    k = KATS["glm_norm_topk"]
    logits = xorshift_vec(5, 3)
    ids, w = orc.route_sigmoid(logits, 3, bias=xorshift_vec(5, 4), norm_topk=True, routed_scale=k["routed_scale"])
    assert abs(float(w.sum()) - k["routed_scale"]) < k["tol"]


def test_boundary_router_is_decided_by_the_fold(orc):
    """helpers.boundary_router: the oracle's logits of experts a and b are the fold's (1 and
    1 + 2^-18) while their exact sums tie, and b, not a, takes the last of the k places under both
    selection rules (the GPU tests use it to reach a router decision that only exact folds settle)."""
    from helpers import boundary_router
    E, H, k = 64, 1024, 8
    x = np.random.default_rng(5).standard_normal(H).astype(np.float32)
    router, a, b, hi = boundary_router(E, H, k, x)
    logits = orc.matmul(x, router.ravel(), 1, H, E).ravel()
    assert logits[a] == np.float32(1.0) and logits[b] == np.float32(1.0 + 2.0 ** -18)
    exact = router.astype(np.float64) @ x.astype(np.float64)
    assert exact[a] == exact[b] == 1.0 + 2.0 ** -18
    for ids, _ in (orc.route_softmax(logits, k), orc.route_sigmoid(logits, k, norm_topk=True)):
        assert sorted(ids) == sorted(hi + [b]) and a not in list(ids)


@pytest.mark.parametrize("k", [2, 10])
def test_tied_boundary_router_is_decided_by_the_fold(orc, k):
    """helpers.tied_boundary_router: the five tied experts' exact sums are equal, the oracle's
    logits are the predicted folds 1 + 2^-23 m_i (all distinct), and the tied expert with the
    largest fold (the highest id, which the midpoint order ranks last) takes the last of the k
    places under both selection rules."""
    from helpers import tied_boundary_router
    E, H = 64, 1024
    x = np.random.default_rng(6).standard_normal(H).astype(np.float32)
    router, tied, folds, hi = tied_boundary_router(E, H, k, x)
    logits = orc.matmul(x, router.ravel(), 1, H, E).ravel()
    assert [logits[e] for e in tied] == folds and len(set(folds)) == len(folds)
    exact = router.astype(np.float64) @ x.astype(np.float64)
    assert all(exact[e] == 1.0 + 2.0 ** -18 for e in tied)
    for ids, _ in (orc.route_softmax(logits, k), orc.route_sigmoid(logits, k, norm_topk=True)):
        assert sorted(ids) == sorted(hi + [tied[-1]])


def test_glm_grouped_kats(orc):
    for c in KATS["glm_grouped"]["cases"]:
        # The KATs rank raw choice values; sigmoid is strictly monotone on them, so feeding the
        # logit = choice through route_sigmoid must give the same ids.
        ids, _ = orc.route_sigmoid(np.array(c["choice"], np.float32), c["k"], norm_topk=False,
                                   n_group=c["n_group"], topk_group=c["topk_group"])
        assert list(ids) == c["ids"]


def test_unique_experts_first_occurrence_order(orc):
    ids = np.array([[5, 2, 9], [2, 7, 5], [1, 9, 3]], np.int32)
    assert list(orc.unique_experts(ids)) == [5, 2, 9, 7, 1, 3]


# ---- experts and layers ------------------------------------------------------------------------
def test_fused_gate_up_matches_separate_bit_exact(orc):
    k = KATS["fused_separate"]
    d, i = k["d"], k["i"]
    gate = xorshift_vec(i * d, 7)
    up = xorshift_vec(i * d, 8)
    down = xorshift_vec(d * i, 9)
    sep = orc.Slot(0, orc.QT.f32(down, d, i), gate=orc.QT.f32(gate, i, d), up=orc.QT.f32(up, i, d))
    fus = orc.Slot(0, orc.QT.f32(down, d, i), gate_up=orc.QT.f32(np.concatenate([gate, up]), 2 * i, d))
    x = xorshift_vec(3 * d, 10)
    ids = np.zeros((3, 1), np.int32)
    w = np.array(k["weights"], np.float32).reshape(3, 1)
    a = orc.apply_single_expert(sep, ids, w, x, d, i, np.zeros(3 * d, np.float32))
    b = orc.apply_single_expert(fus, ids, w, x, d, i, np.zeros(3 * d, np.float32))
    assert bits_equal(a, b)


def _np_expert(x, g, u, dn):
    gg = x @ g.T
    uu = x @ u.T
    h = gg / (1.0 + np.exp(-gg)) * uu
    return h @ dn.T


def test_moe_forward_matches_independent_sum(orc):
    # glm52/moe.rs:1037-1136 pattern: an independent full sum (fp64 numpy) over every routed expert
    d, i, E, s = 64, 32, 6, 3
    experts = {}
    dense = {}
    for e in range(E):
        g = orc.synth_mxfp4(i, d, seed=100 + 3 * e)
        u = orc.synth_mxfp4(i, d, seed=101 + 3 * e)
        dn = orc.synth_mxfp4(d, i, seed=102 + 3 * e)
        experts[e] = orc.Slot(e, dn, gate=g, up=u)
        dense[e] = (g.dense(), u.dense(), dn.dense())
    sg, su, sd = orc.synth_mxfp4(i, d, seed=7), orc.synth_mxfp4(i, d, seed=8), orc.synth_mxfp4(d, i, seed=9)
    shared = orc.Slot(0, sd, gate=sg, up=su)
    rng = np.random.default_rng(3)
    router = (rng.standard_normal((E, d)) * 0.3).astype(np.float32)
    gvec = (rng.standard_normal(d) * 0.1).astype(np.float32)
    x = rng.standard_normal((s, d)).astype(np.float32)
    for fam in (orc.FAMILY_QWEN38, orc.FAMILY_GLM52):
        L = orc.MoeLayer(fam, d, i, E, 3, router, experts, shared=shared,
                         shared_gate=gvec if fam == orc.FAMILY_QWEN38 else None)
        out, ids, w = L.forward(x, s)
        exp = np.zeros((s, d))
        x64 = x.astype(np.float64)
        for t in range(s):
            for j in range(3):
                g, u, dn = dense[int(ids[t, j])]
                exp[t] += w[t, j] * _np_expert(x64[t:t + 1], g, u, dn)[0]
            sh = _np_expert(x64[t:t + 1], sg.dense(), su.dense(), sd.dense())[0]
            if fam == orc.FAMILY_QWEN38:
                sh = sh / (1.0 + np.exp(-(x64[t] @ gvec)))
            exp[t] += sh
        assert rel_l2(out, exp) < 1e-5
        # routing itself: logits by the sequential fold, then the family's router
        lg = L.router_logits(x, s)
        for t in range(s):
            if fam == orc.FAMILY_QWEN38:
                rid, rw = orc.route_softmax(lg[t], 3)
            else:
                rid, rw = orc.route_sigmoid(lg[t], 3)
            assert list(rid) == list(ids[t]) and bits_equal(rw, w[t])


def test_synth_generator_distribution(orc):
    q = orc.synth_mxfp4(256, 1024, seed=42)
    nib = np.concatenate([q.data & 0xF, q.data >> 4])
    hist = np.bincount(nib, minlength=16)
    assert hist.min() > 0.9 * hist.mean() and hist.max() < 1.1 * hist.mean()
    assert q.scale.min() == 119 and q.scale.max() == 123
    g = orc.synth_i4g(64, 256, 32, seed=1)
    assert g.scale.min() >= 0.005 and g.scale.max() < 0.02


# ---- norms and the MoE sublayer -----------------------------------------------------------------
def _np_rms_scale(v, eps):
    # the reference's r: f64 sum of squares in element order, mean rounded to f32, f32 sqrt/divide
    ms = 0.0
    for a in np.asarray(v, np.float32):
        ms += float(a) * float(a)
    return np.float32(1.0) / np.sqrt(np.float32(ms / len(v)) + np.float32(eps))


def test_rmsnorm_1p_kats(orc):
    # qwen38/ops.rs:42-52: a zero weight leaves the normalised vector alone (1.0); the plain norm
    # zeroes it
    assert np.all(np.abs(orc.rmsnorm_1p([2.0] * 4, [0.0] * 4, 1e-6) - 1.0) < 1e-4)
    assert np.all(orc.rmsnorm([2.0] * 4, [0.0] * 4, 1e-6) == 0.0)
    # :55-69 the formula elementwise (f32 mean square as the test writes it)
    v0 = np.array([1.0, -2.0, 3.0, -4.0, 0.5, 0.25], np.float32)
    w = np.array([0.1, -0.2, 0.0, 0.5, -0.75, 1.0], np.float32)
    ms = np.float32(np.sum(v0 * v0, dtype=np.float32) / np.float32(6))
    want = v0 / np.sqrt(ms + np.float32(1e-6)) * (np.float32(1) + w)
    assert np.all(np.abs(orc.rmsnorm_1p(v0, w, 1e-6) - want) < 1e-5)
    # :73-81 1 + w against w
    assert abs(orc.rmsnorm_1p([3.0] * 8, [0.05] * 8, 1e-6)[0] - 1.05) < 1e-4
    assert abs(orc.rmsnorm([3.0] * 8, [0.05] * 8, 1e-6)[0] - 0.05) < 1e-4


def test_rmsnorm_kats(orc):
    # kimi_linear/ops.rs:159-173 against the naive unfused form; :175-182 unit weights give unit RMS
    v = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    w = np.array([1.0, 0.5, 2.0, 1.0], np.float32)
    ms = np.float32(np.sum(v * v, dtype=np.float32) / np.float32(4))
    r = np.float32(1.0) / np.sqrt(ms + np.float32(1e-5))
    assert np.all(np.abs(orc.rmsnorm(v, w, 1e-5) - v * r * w) < 1e-5)
    u = orc.rmsnorm([2.0, -6.0, 3.0, 1.0], [1.0] * 4, 1e-8)
    assert abs(math.sqrt(float(np.mean(u.astype(np.float64) ** 2))) - 1.0) < 1e-4


def test_rmsnorm_closed_form_and_one_plus_relation(orc):
    # bit for bit: r from an f64 sum in order (an f32 sum, a dropped eps or a fused multiply would
    # change the last bits on these rows), and rmsnorm_1p(v, w) == rmsnorm(v, f32(1 + w))
    rng = np.random.default_rng(17)
    for n in (5, 256, 6144, 8192):
        v = (rng.standard_normal(n) * 3).astype(np.float32)
        w = (rng.standard_normal(n) * 0.1).astype(np.float32)
        r = _np_rms_scale(v, 1e-6)
        assert bits_equal(orc.rmsnorm(v, w, 1e-6), v * (r * w))
        assert bits_equal(orc.rmsnorm_1p(v, w, 1e-6), v * (r * (np.float32(1) + w)))
        assert bits_equal(orc.rmsnorm_1p(v, w, 1e-6), orc.rmsnorm(v, np.float32(1) + w, 1e-6))


def test_moe_sublayer_is_residual_plus_forward_of_normalised(orc):
    # qwen38/generate.rs:397-413: x + moe_forward(rmsnorm_1p(x)), not moe_forward(x) + x
    d, i, E, s = 64, 32, 6, 3
    experts = {e: orc.Slot(e, orc.synth_mxfp4(d, i, seed=12 + 3 * e), gate=orc.synth_mxfp4(i, d, seed=10 + 3 * e),
                           up=orc.synth_mxfp4(i, d, seed=11 + 3 * e)) for e in range(E)}
    rng = np.random.default_rng(5)
    router = (rng.standard_normal((E, d)) * 0.3).astype(np.float32)
    L = orc.MoeLayer(orc.FAMILY_QWEN38, d, i, E, 2, router, experts)
    x = (rng.standard_normal((s, d)) * 2).astype(np.float32)
    ln = (rng.standard_normal(d) * 0.1).astype(np.float32)
    got, ids, w = L.sublayer(x, s, ln, 1e-6)
    nrm = orc.rmsnorm_1p(x, ln, 1e-6)
    out, ids2, w2 = L.forward(nrm, s)
    assert np.array_equal(ids, ids2) and bits_equal(w, w2)
    assert bits_equal(got, x + out)
    plain, _, _ = L.forward(x, s)
    assert not np.allclose(got, x + plain)


# ---- K3: Situ activation and the latent MoE ----------------------------------------------------------
def _situ64(g, u, beta, lb):
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    if lb is not None:
        u = lb * np.tanh(u / lb)
    return beta * np.tanh(g / beta) / (1.0 + np.exp(-g)) * u


@pytest.mark.parametrize("gate,up,lb", [([-3.0, -0.5, 0.0, 0.5, 3.0, 10.0], [2.0, -1.0, 4.0, -4.0, 0.1, 30.0], 25.0),
                                        ([-2.0, 0.0, 1.5], [3.0, -2.0, 0.5], None)])
def test_situ_kats(orc, gate, up, lb):
    # kimi_linear/ops.rs:236-260: beta 4, with and without linear_beta, against the formula in fp64
    act = orc.situ(4.0, lb)
    got = np.array([orc.act_combine(act, g, u) for g, u in zip(gate, up)])
    assert np.max(np.abs(got - _situ64(gate, up, 4.0, lb))) < 1e-5


def test_situ_special_values(orc):
    # kimi_linear/ops.rs:262-277: gate 0 gives exactly 0 whatever up is; gate >> beta saturates to beta * up
    act = orc.situ(4.0, 25.0)
    assert orc.act_combine(act, 0.0, 123.0) == 0.0 and orc.act_combine(act, 0.0, -456.0) == 0.0
    assert abs(orc.act_combine(orc.situ(4.0), 1000.0, 2.0) - 8.0) < 1e-3
    # linear_beta saturates up: lb * tanh(u / lb) -> lb for u >> lb
    assert abs(orc.act_combine(orc.situ(4.0, 2.0), 1000.0, 1e4) - 8.0) < 1e-3
    # beta -> inf: beta * tanh(g / beta) -> g, so Situ -> SiLU (a dropped sigmoid or tanh fails this)
    for g, u in ((-2.5, 0.7), (0.3, -1.1), (4.0, 2.0)):
        silu = orc.act_combine(None, g, u)
        assert abs(orc.act_combine(orc.situ(1e4), g, u) - silu) < 1e-5 * max(1.0, abs(silu))
        assert abs(silu - g / (1.0 + math.exp(-g)) * u) < 1e-6


def test_situ_expert_matches_independent_and_differs_from_silu(orc):
    # glm52/moe.rs:842-883: an expert with Situ(4, 25) against an independent fp64 re-derivation
    d, i = 4, 3
    g, u, dn = xorshift_vec(i * d, 5), xorshift_vec(i * d, 6), xorshift_vec(d * i, 7)
    slot = orc.Slot(0, orc.QT.f32(dn, d, i), gate=orc.QT.f32(g, i, d), up=orc.QT.f32(u, i, d))
    x = xorshift_vec(d, 8)
    ids, w = np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32)
    act = orc.situ(4.0, 25.0)
    out = orc.apply_single_expert(slot, ids, w, x, d, i, np.zeros(d, np.float32), act=act)
    x64 = x.astype(np.float64)
    hg = g.reshape(i, d).astype(np.float64) @ x64
    hu = u.reshape(i, d).astype(np.float64) @ x64
    exp = dn.reshape(d, i).astype(np.float64) @ _situ64(hg, hu, 4.0, 25.0)
    assert np.max(np.abs(out - exp)) < 1e-5
    silu = orc.apply_single_expert(slot, ids, w, x, d, i, np.zeros(d, np.float32))
    assert not np.array_equal(out, silu)


def test_situ_fused_gate_up_matches_separate_bit_exact(orc):
    # glm52/moe.rs:885-919: the fused branch's per-element combine agrees with the separate branch's
    d, i = 6, 8
    gate, up, down = xorshift_vec(i * d, 17), xorshift_vec(i * d, 18), xorshift_vec(d * i, 19)
    sep = orc.Slot(0, orc.QT.f32(down, d, i), gate=orc.QT.f32(gate, i, d), up=orc.QT.f32(up, i, d))
    fus = orc.Slot(0, orc.QT.f32(down, d, i), gate_up=orc.QT.f32(np.concatenate([gate, up]), 2 * i, d))
    x = xorshift_vec(3 * d, 20)
    ids = np.zeros((3, 1), np.int32)
    w = np.array([[0.6], [1.3], [-0.4]], np.float32)
    act = orc.situ(4.0, 25.0)
    a = orc.apply_single_expert(sep, ids, w, x, d, i, np.zeros(3 * d, np.float32), act=act)
    b = orc.apply_single_expert(fus, ids, w, x, d, i, np.zeros(3 * d, np.float32), act=act)
    assert bits_equal(a, b)


def _latent_fixture(orc, seed, E=4, H=6, MH=4, I=3, k=2):
    # kimi_k3/moe.rs:232-262's shapes: a sigmoid router with a correction bias over the full width,
    # experts at moe_hidden, projections [MH, H] and [H, MH]
    dense = {}
    experts = {}
    for e in range(E):
        g, u, dn = (xorshift_vec(I * MH, seed + 10 * e + j) for j in range(3))
        experts[e] = orc.Slot(e, orc.QT.f32(dn, MH, I), gate=orc.QT.f32(g, I, MH), up=orc.QT.f32(u, I, MH))
        dense[e] = (g.reshape(I, MH), u.reshape(I, MH), dn.reshape(MH, I))
    router = xorshift_vec(E * H, seed + 100)
    bias = xorshift_vec(E, seed + 101)
    L = orc.MoeLayer(orc.FAMILY_GLM52, H, I, E, k, router, experts, router_bias=bias, norm_topk=False)
    down = xorshift_vec(MH * H, seed + 102).reshape(MH, H)
    up = xorshift_vec(H * MH, seed + 103).reshape(H, MH)
    return L, dense, down, up


def _latent_expected(L, dense, down, up, x, s, norm=None, eps=1e-5, act=None):
    ids, w = L.route(x, s)
    x64 = x.reshape(s, -1).astype(np.float64)
    xl = x64 @ down.astype(np.float64).T
    routed = np.zeros((s, down.shape[0]))
    for t in range(s):
        for j in range(ids.shape[1]):
            g, u, dn = (a.astype(np.float64) for a in dense[int(ids[t, j])])
            hg, hu = g @ xl[t], u @ xl[t]
            h = hg / (1.0 + np.exp(-hg)) * hu if act is None else _situ64(hg, hu, *act)
            routed[t] += w[t, j] * (dn @ h)
    if norm is not None:
        routed = routed / np.sqrt(np.mean(routed ** 2, axis=1, keepdims=True) + eps) * norm.astype(np.float64)
    return routed @ up.astype(np.float64).T, routed, ids, w


def test_latent_moe_matches_independent_without_norm(orc):
    # kimi_k3/moe.rs:232-281: route at full width, down-project, experts at moe_hidden, up-project
    L, dense, down, up = _latent_fixture(orc, 11)
    s = 3
    x = xorshift_vec(s * 6, 50)
    out, ids, w = L.latent(x, s, 4, orc.QT.f32(down.ravel(), 4, 6), orc.QT.f32(up.ravel(), 6, 4))
    exp, _, eids, ew = _latent_expected(L, dense, down, up, x, s)
    assert np.array_equal(ids, eids) and bits_equal(w, ew)
    assert np.max(np.abs(out - exp)) < 1e-5
    # routing is the layer's own (full-width x), not that of the projected x
    rid, _ = orc.route_sigmoid(L.router_logits(x, s)[0], 2, bias=L.router_bias, norm_topk=False)
    assert list(rid) == list(ids[0])


def test_latent_moe_norm_applies_to_the_summed_rows(orc):
    # kimi_k3/moe.rs:283-330: rmsnorm of each token's summed routed output, before up_proj
    L, dense, down, up = _latent_fixture(orc, 23)
    s = 2
    x = xorshift_vec(s * 6, 60)
    norm = np.abs(xorshift_vec(4, 61)) + np.float32(0.5)
    dq, uq = orc.QT.f32(down.ravel(), 4, 6), orc.QT.f32(up.ravel(), 6, 4)
    out, _, _ = L.latent(x, s, 4, dq, uq, norm=norm, eps=1e-5)
    exp, routed, _, _ = _latent_expected(L, dense, down, up, x, s, norm=norm)
    unnormed = _latent_expected(L, dense, down, up, x, s)[1]
    assert not np.allclose(routed, unnormed)
    assert np.max(np.abs(out - exp)) < 1e-5
    # per-expert normalisation would be a different (wrong) answer
    plain, _, _ = L.latent(x, s, 4, dq, uq)
    assert not np.allclose(out, plain)


def test_latent_moe_with_situ(orc):
    L, dense, down, up = _latent_fixture(orc, 31)
    s = 3
    x = xorshift_vec(s * 6, 70)
    out, _, _ = L.latent(x, s, 4, orc.QT.f32(down.ravel(), 4, 6), orc.QT.f32(up.ravel(), 6, 4),
                         act=orc.situ(4.0, 25.0))
    exp, _, _, _ = _latent_expected(L, dense, down, up, x, s, act=(4.0, 25.0))
    assert np.max(np.abs(out - exp)) < 1e-5


def test_latent_moe_identity_projections_equal_routed_forward(orc):
    # with moe_hidden == hidden and identity projections the latent MoE is the routed part of
    # moe_forward exactly (same routing, same per-expert accumulation order)
    d, i, E, s, k = 64, 32, 6, 3, 3
    experts = {e: orc.Slot(e, orc.synth_mxfp4(d, i, seed=40 + 3 * e), gate=orc.synth_mxfp4(i, d, seed=41 + 3 * e),
                           up=orc.synth_mxfp4(i, d, seed=42 + 3 * e)) for e in range(E)}
    rng = np.random.default_rng(9)
    router = (rng.standard_normal((E, d)) * 0.3).astype(np.float32)
    L = orc.MoeLayer(orc.FAMILY_GLM52, d, i, E, k, router, experts, routed_scale=2.5)
    x = rng.standard_normal((s, d)).astype(np.float32)
    eye = orc.QT.f32(np.eye(d, dtype=np.float32).ravel(), d, d)
    lat, lid, lw = L.latent(x, s, d, eye, eye)
    fwd, fid, fw = L.forward(x, s)
    assert np.array_equal(lid, fid) and bits_equal(lw, fw)
    assert np.array_equal(lat, fwd)
