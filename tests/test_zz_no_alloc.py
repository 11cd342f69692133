"""The allocation-free entry point (rbt_moe_forward_noalloc_d) against rbt_moe_forward_d, through
the C ABI: the same kernels on buffers carved out of the device's fixed scratch array, so ids,
weights and outputs must be bit-identical. Two calls in a row (the second with fewer tokens, so it
runs on what the first left in the array), the one-token decode path, and the size limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pair(ctx, x, S, H, k, noalloc):
    import torch
    out = torch.full((S * H,), float("nan"), dtype=torch.float32, device="cuda")
    ids = torch.full((S * k,), -7, dtype=torch.int32, device="cuda")
    w = torch.full((S * k,), float("nan"), dtype=torch.float32, device="cuda")
    (ctx.moe_forward_noalloc if noalloc else ctx.moe_forward)(0, x, S, out, ids, w)
    return out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()


def _check(ctx, x, S, H, k):
    a = _pair(ctx, x, S, H, k, noalloc=False)
    b = _pair(ctx, x, S, H, k, noalloc=True)
    assert np.array_equal(a[1], b[1])
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    assert np.array_equal(a[2].view(np.uint32), b[2].view(np.uint32))
    assert np.all(np.isfinite(b[0]))


def test_noalloc_matches_allocating_entry(ctx):
    import torch
    import rabbit_amd as R
    import rabbit_amd.workloads as W
    cfg = W.CONFIGS["c1"]
    W.build_layer(ctx, cfg, layer=0, seed=1000)
    H, k = cfg.hidden, cfg.topk
    x = torch.from_numpy(W.tokens(cfg, 16, 31)).cuda()
    for S in (8, 2):  # two calls in a row, the second smaller
        print(f"noalloc c1 S={S}", flush=True)
        _check(ctx, x[:S].contiguous(), S, H, k)
    for t in range(4):  # one-token decode (router launch, balanced gate/up and down)
        print(f"noalloc c1 S=1 token {t}", flush=True)
        _check(ctx, x[t:t + 1].contiguous(), 1, H, k)
    # a call whose buffers do not fit the fixed array is refused, and the context stays usable
    big = torch.from_numpy(W.tokens(cfg, 512, 32)).cuda()
    out = torch.empty(512 * H, dtype=torch.float32, device="cuda")
    with pytest.raises(R.RbtError) as ei:
        ctx.moe_forward_noalloc(0, big, 512, out)
    assert ei.value.status == R.abi.RBT_E_UNSUPPORTED
    _check(ctx, x[:3].contiguous(), 3, H, k)


def test_noalloc_small_layers(ctx, orc):
    """GLM (grouped int4) and K3 routing through the per-pair kernels at small shapes."""
    import torch
    import rabbit_amd as R
    from test_gpu_moe import _small_layer
    from helpers import normal
    for family, kind, lb in ((1, R.QT_I4_GROUPED, False), (2, R.QT_MXFP4, True)):
        H, I, E, k = 256, 128, 24, 4
        _small_layer(ctx, orc, family, kind, H, I, E, k, seed=40 + family, logit_bias=lb)
        x = torch.from_numpy(normal((6, H), 9 + family)).cuda()
        for S in (6, 1):
            print(f"noalloc family={family} S={S}", flush=True)
            _check(ctx, x[:S].contiguous(), S, H, k)
