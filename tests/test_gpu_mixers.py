"""GPU parity of Qwen 3.8's token mixers (rbt_gdn_step_d, rbt_gqa_step_d) against the oracle's
restatement of qwen38/gdn.rs:142-196 (+ kimi_linear/short_conv.rs:58-85) and qwen38/generate.rs:226-255
(oracle/rabbit_oracle_mixers.c), token after token with the carried state (GDN conv history and
delta-rule matrices, GQA KV cache) on both sides.

Bar: every token's output and the carried state within 1e-5 relative L2 of the oracle (fp32
accumulation in a different order; the reference's transcendentals are libm's, the device's are
fp64 rounded to fp32).
"""
import numpy as np
import pytest

from helpers import rel_l2

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


@pytest.mark.parametrize("n_v,n_k,d_k,d_v,steps,K", [(4, 2, 16, 8, 6, 4), (8, 8, 32, 64, 4, 4),
                                                    (128, 16, 128, 128, 4, 4), (8, 2, 32, 64, 5, 3),
                                                    (16, 4, 64, 512, 3, 4), (4, 2, 16, 8, 5, 2),
                                                    (4, 2, 16, 8, 7, 5)])
def test_gdn_step_matches_oracle(ctx, orc, n_v, n_k, d_k, d_v, steps, K):
    """Small shapes and Qwen 3.8's (128 V heads over 16 K heads, 128 x 128 state, conv_dim 20480), with
    conv kernels 4, 3 and 2 (compiled for their size) and 5 (the conv kernel for any size); the head
    kernel's row count per thread is fixed at 8 (Qwen 3.8) and 16 (head_v_dim 512) and runtime in the
    other cases."""
    import torch
    rng = np.random.default_rng(n_v * 7 + d_k)
    key_dim = n_k * d_k
    conv_dim = 2 * key_dim + n_v * d_v
    conv_w = (rng.standard_normal((conv_dim, K)) * 0.5).astype(np.float32)
    a_log = (rng.standard_normal(n_v) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(n_v) * 0.5).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(d_v)).astype(np.float32)
    st = orc.GdnState(n_v, n_k, d_k, d_v, K)
    d_conv = torch.zeros(conv_dim * (K - 1), dtype=torch.float32, device="cuda")
    d_states = torch.zeros(n_v * d_k * d_v, dtype=torch.float32, device="cuda")
    out = torch.empty(n_v * d_v, dtype=torch.float32, device="cuda")
    tw, ta, tdt, tnw = _t(conv_w), _t(a_log), _t(dt), _t(nw)
    for step in range(steps):
        x = rng.standard_normal(conv_dim).astype(np.float32)
        z = rng.standard_normal(n_v * d_v).astype(np.float32)
        a = rng.standard_normal(n_v).astype(np.float32)
        b = rng.standard_normal(n_v).astype(np.float32)
        want = orc.gdn_step(st, x, conv_w, z, a, b, a_log, dt, nw, 1e-6)
        ctx.gdn_step(n_v, n_k, d_k, d_v, tw, ta, tdt, tnw, 1e-6, d_conv, d_states, _t(x), _t(z), _t(a), _t(b), out,
                     kernel=K)
        got = out.cpu().numpy()
        assert rel_l2(got, want) < RTOL, (step, rel_l2(got, want))
        assert np.array_equal(d_conv.cpu().numpy(), st.conv), step  # the history is a copy of inputs
        assert rel_l2(d_states.cpu().numpy(), st.heads) < RTOL, step


def _gqa_case(ctx, orc, n_heads, n_kv, hd, rope_dim, positions, prefill=0, seed=0):
    import torch
    rng = np.random.default_rng(seed + hd + positions)
    theta, scale, eps = 1e7, 1.0 / np.sqrt(hd), 1e-6
    qn = (0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (0.1 * rng.standard_normal(hd)).astype(np.float32)
    cap = prefill + positions
    kv = orc.KvCache(n_kv, hd, cap)
    if prefill:
        # a long history already in the cache (normalised, rotated keys and raw values)
        kv.k[:prefill] = rng.standard_normal((prefill, n_kv * hd)).astype(np.float32)
        kv.v[:prefill] = rng.standard_normal((prefill, n_kv * hd)).astype(np.float32)
        kv.len = prefill
    d_kc, d_vc = _t(kv.k), _t(kv.v)
    tqn, tkn = _t(qn), _t(kn)
    out = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
    worst = 0.0
    for i in range(positions):
        pos = prefill + i
        qg = rng.standard_normal(2 * n_heads * hd).astype(np.float32)
        k = rng.standard_normal(n_kv * hd).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        want = orc.gqa_step(kv, qg, k, v, n_heads, qn, kn, eps, rope_dim, theta, scale)
        ctx.gqa_step(n_heads, n_kv, hd, rope_dim, theta, scale, eps, tqn, tkn, d_kc, d_vc, cap, pos, _t(qg), _t(k),
                     _t(v), out)
        got = out.cpu().numpy()
        e = rel_l2(got, want)
        worst = max(worst, e)
        assert e < RTOL, (pos, e)
        assert rel_l2(d_kc.cpu().numpy()[pos], kv.k[pos]) < RTOL, pos
        assert np.array_equal(d_vc.cpu().numpy()[pos], kv.v[pos]), pos
    return worst


@pytest.mark.parametrize("n_heads,n_kv,hd,rope_dim,positions", [(8, 2, 64, 16, 9), (64, 4, 256, 64, 70),
                                                               (8, 2, 512, 320, 5), (4, 1, 1024, 1024, 3),
                                                               (4, 2, 128, 0, 3)])
def test_gqa_step_matches_oracle(ctx, orc, n_heads, n_kv, hd, rope_dim, positions):
    """Positions 0..positions-1 from an empty cache (70 positions: two score chunks); the second case is
    Qwen 3.8's shape (64 query heads over 4 KV heads, head_dim 256, 64 rotated dims, theta 1e7); head
    dims 512 and 1024 take two and four entries per thread (all 1024 rotated), and rope_dim 0 none."""
    worst = _gqa_case(ctx, orc, n_heads, n_kv, hd, rope_dim, positions)
    print(f"gqa {n_heads}/{n_kv}x{hd}: worst rel-L2 {worst:.2e}")


@pytest.mark.parametrize("prefill", [2000, 4000, 6200, 30000])
def test_gqa_step_long_cache(ctx, orc, prefill):
    """Qwen 3.8's shape at positions prefill..prefill+2 of a prefilled cache (32, 63, 97 and 469
    score chunks: the combine's sixteen-chunk batches with and without a remainder, and more chunks
    than threads; RoPE angles up to 30002 radians)."""
    worst = _gqa_case(ctx, orc, 64, 4, 256, 64, 3, prefill=prefill, seed=5)
    print(f"gqa long cache at {prefill}: worst rel-L2 {worst:.2e}")


def test_mixer_errors(ctx, orc):
    import rabbit_amd as R
    import torch
    z = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    with pytest.raises(R.RbtError) as e:  # position past the cache
        ctx.gqa_step(8, 2, 64, 16, 1e7, 0.125, 1e-6, z, z, z, z, 4, 4, z, z, z, z)
    assert e.value.status == R.abi.RBT_E_INVALID
    with pytest.raises(R.RbtError) as e:  # head_v_dim 6 is not a multiple of 4
        ctx.gdn_step(2, 1, 8, 6, z, z, z, z, 1e-6, z, z, z, z, z, z, z)
    assert e.value.status == R.abi.RBT_E_UNSUPPORTED
    with pytest.raises(R.RbtError) as e:  # V heads not a multiple of K heads
        ctx.gdn_step(3, 2, 8, 8, z, z, z, z, 1e-6, z, z, z, z, z, z, z)
    assert e.value.status == R.abi.RBT_E_INVALID
