"""Pins the oracle's restatement of Qwen 3.8's token mixers (oracle/rabbit_oracle_mixers.c).

The reference's own tests for these functions are restated here with their literals
(qwen38/gdn.rs:234-424, qwen38/attention.rs:228-391), and the whole mixer steps are checked against
float64 transcriptions of the formulas written independently of the oracle (numpy, below) on random
inputs, so a dropped term, a swapped operand or a wrong head mapping fails one of them.
"""
import numpy as np
import pytest

from helpers import rel_l2


# ---- independent float64 transcriptions ----------------------------------------------------------
def _silu64(x):
    return x / (1.0 + np.exp(-x))


def _ramp(n, seed):
    """qwen38/gdn.rs:242-244: ((i * 37 + seed) % 23 - 11) / 5."""
    return np.array([(((i * 37 + seed) % 23) - 11.0) / 5.0 for i in range(n)], np.float32)


def _gdn64(states, qkv_pre, conv_hist, conv_w, z, a, b, a_log, dt_bias, nw, eps, n_v, n_k, d_k, d_v, K):
    """One GDN token in float64 from the reference's Python formulation (the transformers loop that
    qwen38/gdn.rs:8-20 quotes): conv + SiLU, split, l2 norms, decay, delta rule, gated RMSNorm.
    states [n_v, d_k, d_v] and conv_hist [conv_dim, K-1] are float64 and updated in place."""
    key_dim = n_k * d_k
    x = qkv_pre.astype(np.float64)
    full = np.concatenate([conv_hist, x[:, None]], axis=1)          # [conv_dim, K]
    conv = (full * conv_w.reshape(-1, K).astype(np.float64)).sum(1)
    conv_hist[:, :-1] = conv_hist[:, 1:]
    conv_hist[:, -1] = x
    act = _silu64(conv)
    q, k, v = act[:key_dim].reshape(n_k, d_k), act[key_dim:2 * key_dim].reshape(n_k, d_k), act[2 * key_dim:]
    q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-6) / np.sqrt(d_k)
    k = k / np.maximum(np.linalg.norm(k, axis=1, keepdims=True), 1e-6)
    out = np.zeros(n_v * d_v)
    rep = n_v // n_k
    for h in range(n_v):
        g = np.exp(-np.exp(np.float64(a_log[h])) * np.log1p(np.exp(np.float64(a[h]) + dt_bias[h])))
        beta = 1.0 / (1.0 + np.exp(-np.float64(b[h])))
        S = states[h] * g
        kv_mem = S.T @ k[h // rep]
        delta = (v[h * d_v:(h + 1) * d_v] - kv_mem) * beta
        S = S + np.outer(k[h // rep], delta)
        states[h] = S
        o = S.T @ q[h // rep]
        o = o / np.sqrt(np.mean(o * o) + eps) * nw.astype(np.float64)
        out[h * d_v:(h + 1) * d_v] = o * _silu64(z[h * d_v:(h + 1) * d_v].astype(np.float64))
    return out


def _gqa64(qg, k_in, v_in, kc, vc, pos, n_heads, n_kv, hd, qn, kn, eps, rope_dim, theta, scale):
    """One GQA token in float64 (transformers' Qwen3_5MoeAttention.forward as qwen38/attention.rs:1-45
    describes it): per-head q/gate split, (1+w) RMSNorm, rotate_half RoPE on the first rope_dim dims,
    append, softmax(q k^T * scale) v with query head h reading KV head h / (n_heads / n_kv), gate."""
    qg = qg.astype(np.float64).reshape(n_heads, 2, hd)
    q, gate = qg[:, 0], qg[:, 1]
    k = k_in.astype(np.float64).reshape(n_kv, hd)

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps) * (1.0 + w.astype(np.float64))

    def rope(x):
        half = rope_dim // 2
        f = pos / theta ** (2.0 * np.arange(half) / rope_dim)
        c, s = np.cos(np.concatenate([f, f])), np.sin(np.concatenate([f, f]))
        r = x[:, :rope_dim]
        rot = np.concatenate([-r[:, half:], r[:, :half]], axis=1)
        return np.concatenate([r * c + rot * s, x[:, rope_dim:]], axis=1)

    q, k = rope(norm(q, qn)), rope(norm(k, kn))
    kc[pos] = k.reshape(-1)
    vc[pos] = v_in.astype(np.float64)
    K = kc[:pos + 1].reshape(pos + 1, n_kv, hd)
    V = vc[:pos + 1].reshape(pos + 1, n_kv, hd)
    out = np.zeros((n_heads, hd))
    rep = n_heads // n_kv
    for h in range(n_heads):
        s = K[:, h // rep] @ q[h] * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[:, h // rep]
    return (out / (1.0 + np.exp(-gate))).reshape(-1)


# ---- GDN: the reference's tests ------------------------------------------------------------------
def test_gdn_step_matches_the_reference_recurrence(orc):
    """qwen38/gdn.rs:233-279: KdaState::step with a broadcast decay equals a literal transcription
    of torch_recurrent_gated_delta_rule's loop body, token after token (1e-5)."""
    d_k, d_v = 8, 6
    s = np.zeros((d_k, d_v), np.float32)
    ref = np.zeros(d_k * d_v, np.float32)
    for t in range(5):
        q, k = orc.gdn_prepare_qk(_ramp(d_k, t), _ramp(d_k, t + 7))
        v = _ramp(d_v, t + 13)
        g = orc.gdn_alpha(0.3, -0.4 + t * 0.2, 0.7)
        beta = orc.sigmoid(0.25 * t - 0.5)
        got = orc.kda_step(s, q, k, v, g, beta)
        # reference_step, element by element in float32 (gdn.rs:247-274)
        ref *= np.float32(g)
        kv_mem = np.zeros(d_v, np.float32)
        for i in range(d_k):
            for j in range(d_v):
                kv_mem[j] += ref[i * d_v + j] * k[i]
        delta = (v - kv_mem) * np.float32(beta)
        for i in range(d_k):
            for j in range(d_v):
                ref[i * d_v + j] += k[i] * delta[j]
        want = np.zeros(d_v, np.float32)
        for i in range(d_k):
            for j in range(d_v):
                want[j] += ref[i * d_v + j] * q[i]
        assert np.max(np.abs(got - want)) < 1e-5, t


@pytest.mark.parametrize("a_log,a,dt", [(0.0, 0.0, 0.0), (0.5, -1.0, 0.7), (2.0, 3.0, -0.2), (-1.0, 0.4, 1.5)])
def test_gdn_decay_formula(orc, a_log, a, dt):
    """qwen38/gdn.rs:283-302: alpha = exp(-exp(a_log) softplus(a + dt_bias)), within (0, 1]."""
    got = orc.gdn_alpha(a_log, a, dt)
    x = a + dt
    want = np.exp(-np.exp(a_log) * (max(x, 0.0) + np.log1p(np.exp(-abs(x)))))
    assert abs(got - want) < 1e-6 and 0.0 < got <= 1.0


def test_gdn_prepare_qk_normalises_both_and_scales_only_the_query(orc):
    """qwen38/gdn.rs:329-340."""
    d_k = 16
    q, k = orc.gdn_prepare_qk(np.full(d_k, 3.0), np.full(d_k, 4.0))
    assert abs(np.linalg.norm(k) - 1.0) < 1e-4
    assert abs(np.linalg.norm(q) - 1.0 / np.sqrt(d_k)) < 1e-4


def test_gdn_output_gate_uses_silu_not_sigmoid(orc):
    """qwen38/gdn.rs:345-365: silu(0) = 0 zeroes the head; silu(12) ~ 12 scales the normalised 1."""
    w = np.ones(4, np.float32)
    assert np.all(np.abs(orc.gdn_output_gate(np.full(4, 2.0), w, np.zeros(4), 1e-6)) < 1e-6)
    assert np.all(orc.gdn_output_gate(np.full(4, 2.0), w, np.full(4, 12.0), 1e-6) > 11.0)


def _gdn_small(orc, qkv, n_v, n_k, d_k, d_v):
    state = orc.GdnState(n_v, n_k, d_k, d_v)
    z = np.full(n_v * d_v, 2.0, np.float32)
    a, b = np.full(n_v, 0.1, np.float32), np.full(n_v, 0.2, np.float32)
    a_log, dt = np.zeros(n_v, np.float32), np.full(n_v, 0.5, np.float32)
    return orc.gdn_step_token(state, qkv, z, a, b, a_log, dt, np.ones(d_v, np.float32), 1e-6)


def test_gdn_value_heads_read_their_own_key_head(orc):
    """qwen38/gdn.rs:369-402: 4 V heads over 2 K heads; changing K head 1 changes V heads 2, 3 only
    (repeat_interleave blocks, gdn.rs:62-65), and the split is q | k | v in that order."""
    n_v, n_k, d_k, d_v = 4, 2, 4, 3
    key_dim = n_k * d_k
    base = _ramp(2 * key_dim + n_v * d_v, 1)
    base[key_dim:key_dim + d_k] = 0.5 + np.arange(d_k) * 0.1
    before = _gdn_small(orc, base, n_v, n_k, d_k, d_v)
    bad = base.copy()
    bad[key_dim + d_k:key_dim + 2 * d_k] += 3.0
    after = _gdn_small(orc, bad, n_v, n_k, d_k, d_v)
    for h in range(n_v):
        changed = np.any(np.abs(before[h * d_v:(h + 1) * d_v] - after[h * d_v:(h + 1) * d_v]) > 1e-6)
        assert changed == (h // (n_v // n_k) == 1), h


def test_gdn_state_carries_across_tokens(orc):
    """qwen38/gdn.rs:404-423: the same token twice gives two outputs; a fresh state reproduces the
    first exactly."""
    n_v, n_k, d_k, d_v = 2, 1, 4, 3
    qkv = _ramp(2 * n_k * d_k + n_v * d_v, 5)
    state = orc.GdnState(n_v, n_k, d_k, d_v)
    args = (np.full(n_v * d_v, 1.5), np.full(n_v, 0.3), np.full(n_v, 0.4), np.full(n_v, 0.2), np.full(n_v, 0.1),
            np.ones(d_v), 1e-6)
    first = orc.gdn_step_token(state, qkv, *args)
    second = orc.gdn_step_token(state, qkv, *args)
    assert not np.array_equal(first, second)
    again = orc.gdn_step_token(orc.GdnState(n_v, n_k, d_k, d_v), qkv, *args)
    assert np.array_equal(first, again)


def test_short_conv_is_causal_over_the_last_kernel_inputs(orc):
    """kimi_linear/short_conv.rs:58-85: out[c] = w[c,0] x[t-3] + ... + w[c,3] x[t] (zero history
    first), checked against float64 over five steps."""
    C, K = 5, 4
    rng = np.random.default_rng(3)
    w = rng.standard_normal((C, K)).astype(np.float32)
    st = orc.GdnState(1, 1, 1, 1, K)
    st.conv_dim = C
    st.conv = np.zeros(C * (K - 1), np.float32)
    xs = rng.standard_normal((5, C)).astype(np.float32)
    for t in range(5):
        got = orc.short_conv_step(st, xs[t], w)
        hist = np.zeros((K, C))
        for j in range(K):
            if t - (K - 1) + j >= 0:
                hist[j] = xs[t - (K - 1) + j]
        want = (w.T.astype(np.float64) * hist).sum(0)
        assert np.max(np.abs(got - want)) < 1e-5, t


@pytest.mark.parametrize("n_v,n_k,d_k,d_v", [(4, 2, 16, 8), (16, 2, 32, 32)])
def test_gdn_step_against_float64(orc, n_v, n_k, d_k, d_v):
    """Several tokens of conv + step_token against the float64 transcription above."""
    K = 4
    rng = np.random.default_rng(n_v + d_k)
    key_dim = n_k * d_k
    conv_dim = 2 * key_dim + n_v * d_v
    conv_w = (rng.standard_normal((conv_dim, K)) * 0.5).astype(np.float32)
    a_log = rng.standard_normal(n_v).astype(np.float32) * 0.5
    dt = rng.standard_normal(n_v).astype(np.float32) * 0.5
    nw = (1.0 + 0.1 * rng.standard_normal(d_v)).astype(np.float32)
    st = orc.GdnState(n_v, n_k, d_k, d_v, K)
    s64 = np.zeros((n_v, d_k, d_v))
    h64 = np.zeros((conv_dim, K - 1))
    for t in range(6):
        x = rng.standard_normal(conv_dim).astype(np.float32)
        z = rng.standard_normal(n_v * d_v).astype(np.float32)
        a = rng.standard_normal(n_v).astype(np.float32)
        b = rng.standard_normal(n_v).astype(np.float32)
        got = orc.gdn_step(st, x, conv_w, z, a, b, a_log, dt, nw, 1e-6)
        want = _gdn64(s64, x, h64, conv_w, z, a, b, a_log, dt, nw, 1e-6, n_v, n_k, d_k, d_v, K)
        assert rel_l2(got, want) < 1e-5, t


# ---- GQA: the reference's tests ------------------------------------------------------------------
def _ramp_a(n):
    """qwen38/attention.rs:247-249: ((i * 37 % 19) - 9) / 4."""
    return np.array([((i * 37 % 19) - 9.0) / 4.0 for i in range(n)], np.float32)


@pytest.mark.parametrize("pos", [0, 1, 7, 1000])
def test_rope_half_matches_the_cos_sin_formula(orc, pos):
    """qwen38/attention.rs:231-265: q * cat(cos, cos) + rotate_half(q) * cat(sin, sin) (1e-4)."""
    hd, rd, theta = 256, 64, 1e7
    v = _ramp_a(hd)
    got = orc.rope_half(v, rd, pos, theta)
    half = rd // 2
    f = np.array([pos / theta ** (2.0 * j / rd) for j in range(half)])
    c, s = np.cos(np.concatenate([f, f])), np.sin(np.concatenate([f, f]))
    rot = np.concatenate([-v[half:rd], v[:half]])
    want = np.concatenate([v[:rd] * c + rot * s, v[rd:]])
    assert np.max(np.abs(got - want)) < 1e-4


def test_rope_half_identity_at_zero_and_tail_untouched(orc):
    """qwen38/attention.rs:268-279 and :284-295 (pairs (j, j + half) keep their norm)."""
    v = _ramp_a(256)
    assert np.array_equal(orc.rope_half(v, 64, 0, 1e7), v)
    r = orc.rope_half(v, 64, 13, 1e7)
    assert np.array_equal(r[64:], v[64:]) and not np.array_equal(r[:64], v[:64])
    r5 = orc.rope_half(v[:64], 64, 5, 1e7)
    for j in range(32):
        assert abs((v[j] ** 2 + v[j + 32] ** 2) - (r5[j] ** 2 + r5[j + 32] ** 2)) < 1e-3


def _one_pos(orc, qg, k, v, n_heads, n_kv, hd):
    kv = orc.KvCache(n_kv, hd, 1)
    return orc.gqa_step(kv, qg, k, v, n_heads, np.zeros(hd), np.zeros(hd), 1e-6, 0, 1e7, 1.0)


def test_gqa_query_and_gate_split_per_head(orc):
    """qwen38/attention.rs:299-316: q_proj's row is [q_0, gate_0, q_1, gate_1, ...]. At one position
    the context is the value row, so ctx_h = v * sigmoid(gate_h) reads head h's own gate slice."""
    n_heads, hd = 4, 3
    qg = np.concatenate([np.concatenate([np.full(hd, 10.0 * h), np.full(hd, h - 1.5)]) for h in range(n_heads)])
    v = np.array([7.0, 8.0, 9.0], np.float32)
    ctx = _one_pos(orc, qg, np.ones(hd), v, n_heads, 1, hd)
    for h in range(n_heads):
        assert np.allclose(ctx[h * hd:(h + 1) * hd], v / (1.0 + np.exp(-(h - 1.5))), atol=1e-6), h


def test_gqa_attend_kats(orc):
    """qwen38/attention.rs:333-360: one cached position returns its value; two equal scores average."""
    kc = np.array([[1.0, 0.0, 0.0, 0.0]], np.float32)
    vc = np.array([[7.0, 8.0, 9.0, 10.0]], np.float32)
    assert np.array_equal(orc.gqa_attend(np.full(4, 0.5), kc, vc, 1, 4, 0.5), vc[0])
    kc = np.zeros((2, 2), np.float32)
    vc = np.array([[0.0, 0.0], [4.0, 8.0]], np.float32)
    assert np.array_equal(orc.gqa_attend(np.ones(2), kc, vc, 1, 2, 1.0), np.array([2.0, 4.0], np.float32))


def test_gqa_query_heads_map_onto_contiguous_kv_blocks(orc):
    """qwen38/attention.rs:365-379: 8 query heads over 2 KV heads: heads 0-3 read KV head 0."""
    kc = np.array([[1.0, 0.0, 1.0, 0.0]], np.float32)
    vc = np.array([[1.0, 1.0, 9.0, 9.0]], np.float32)
    out = orc.gqa_attend(np.ones(16), kc, vc, 2, 2, 1.0)
    for h in range(8):
        assert np.array_equal(out[2 * h:2 * h + 2], [1.0, 1.0] if h < 4 else [9.0, 9.0]), h


def test_gqa_output_gate_is_sigmoid(orc):
    """qwen38/attention.rs:381-390: ctx * sigmoid(gate): gate 0 halves, 10 keeps, -10 zeroes."""
    hd = 3
    qg = np.concatenate([np.zeros(hd), np.array([0.0, 10.0, -10.0])])
    ctx = _one_pos(orc, qg, np.zeros(hd), np.full(hd, 2.0), 1, 1, hd)
    assert abs(ctx[0] - 1.0) < 1e-6 and abs(ctx[1] - 2.0) < 1e-3 and abs(ctx[2]) < 1e-3


@pytest.mark.parametrize("n_heads,n_kv,hd,rope_dim,steps", [(8, 2, 64, 16, 9), (16, 4, 256, 64, 5)])
def test_gqa_step_against_float64(orc, n_heads, n_kv, hd, rope_dim, steps):
    """Tokens at positions 0..steps-1 (each attending over everything cached) against float64."""
    rng = np.random.default_rng(hd + steps)
    qn, kn = (0.1 * rng.standard_normal(hd)).astype(np.float32), (0.1 * rng.standard_normal(hd)).astype(np.float32)
    kv = orc.KvCache(n_kv, hd, steps)
    kc64, vc64 = np.zeros((steps, n_kv * hd)), np.zeros((steps, n_kv * hd))
    for pos in range(steps):
        qg = rng.standard_normal(2 * n_heads * hd).astype(np.float32)
        k = rng.standard_normal(n_kv * hd).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        got = orc.gqa_step(kv, qg, k, v, n_heads, qn, kn, 1e-6, rope_dim, 1e7, 1.0 / np.sqrt(hd))
        want = _gqa64(qg, k, v, kc64, vc64, pos, n_heads, n_kv, hd, qn, kn, 1e-6, rope_dim, 1e7, 1.0 / np.sqrt(hd))
        assert rel_l2(got, want) < 1e-5, pos
