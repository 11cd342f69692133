"""GPU checks of the MXFP4 expert loader (ExpertCache::ensure_loaded with ExpertNaming::Qwen38Mxfp4 /
KimiK3Mxfp4, expert_cache.rs:93-208,1227-1256): experts read verbatim from safetensors shards into
the HBM pool run the layer exactly as experts put from host memory, the reference's hand-encoded
fixture bytes decode to its expected values, and shape or name errors are reported without a
half-loaded expert."""
import ctypes as C
import time

import numpy as np
import pytest

from helpers import bits_equal, normal, rel_l2, write_safetensors

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def _qwen_names(layer, eid):
    p = f"model.layers.{layer}.mlp.experts.{eid}."
    return [p + m for m in ("gate_proj", "up_proj", "down_proj")]


def _write_qwen_checkpoint(d, orc, layer, E, H, I, seed, nshards=2):
    """Experts 0..E-1 of `layer` in Qwen 3.8's MXFP4 naming over nshards files, plus unrelated
    tensors; returns the oracle slots."""
    experts, per_shard = {}, [[] for _ in range(nshards)]
    for e in range(E):
        mats = [orc.synth_mxfp4(I, H, seed + 3 * e), orc.synth_mxfp4(I, H, seed + 3 * e + 1),
                orc.synth_mxfp4(H, I, seed + 3 * e + 2)]
        experts[e] = orc.Slot(e, mats[2], gate=mats[0], up=mats[1])
        for name, q in zip(_qwen_names(layer, e), mats):
            per_shard[e % nshards] += [(name + ".weight", "U8", [q.rows, (q.cols + 1) // 2], q.data.tobytes()),
                                       (name + ".weight_scale", "U8", [q.rows, (q.cols + 31) // 32],
                                        q.scale.tobytes())]
    per_shard[0].append((f"model.layers.{layer}.mlp.gate.weight", "F32", [E, H], normal((E, H), 1).tobytes()))
    for s in range(nshards):
        write_safetensors(d / f"model-{s + 1:05d}-of-{nshards:05d}.safetensors", per_shard[s],
                          metadata={"format": "pt"})
    return experts


@pytest.mark.parametrize("S", [1, 3])
def test_loaded_checkpoint_runs_the_layer(ctx, orc, tmp_path, S):
    import rabbit_amd as R
    H, I, E, k, layer = 256, 128, 16, 4, 7
    experts = _write_qwen_checkpoint(tmp_path, orc, layer, E, H, I, seed=300)
    sh = R.Shards(str(tmp_path))
    ctx.pool_load_mxfp4(sh, R.NAMING_QWEN38_MXFP4, layer, range(E), H, I)
    router = normal((E, H), 2, 0.05)
    ctx.moe_layer_set(layer, R.FAMILY_QWEN38, H, I, E, k, router)
    L = orc.MoeLayer(orc.FAMILY_QWEN38, H, I, E, k, router, experts)
    x = normal((S, H), 3 + S)
    exp, eids, ew = L.forward(x, S)
    out = np.empty(S * H, np.float32)
    ids = np.empty(S * k, np.int32)
    ctx.moe_forward(layer, x, S, out, ids)
    assert np.array_equal(ids.reshape(S, k), eids)
    assert rel_l2(out, exp) < RTOL
    # the same experts put from host memory give the same result bit for bit
    for e in range(E):
        s = experts[e]
        ctx.pool_put(layer + 1, R.Slot(e, R.QT.mxfp4(s.down.data, s.down.scale, H, I),
                                       gate=R.QT.mxfp4(s.gate.data, s.gate.scale, I, H),
                                       up=R.QT.mxfp4(s.up.data, s.up.scale, I, H)))
    ctx.moe_layer_set(layer + 1, R.FAMILY_QWEN38, H, I, E, k, router)
    out2 = np.empty(S * H, np.float32)
    ctx.moe_forward(layer + 1, x, S, out2)
    assert bits_equal(out, out2)


def test_k3_naming_hand_encoded_bytes(ctx, orc, tmp_path):
    # expert_cache.rs:1556-1566: w1 row 0 packed low nibble first as 0xB2, 0x87 with scale byte 127
    # decodes to [1.0, -1.5, 6.0, -0.0]
    import rabbit_amd as R
    import rabbit_amd.abi as A
    import torch
    H, I, layer = 64, 8, 3
    p = f"language_model.model.layers.{layer}.block_sparse_moe.experts.0."
    w1 = np.zeros(I * H // 2, np.uint8)
    w1[0], w1[1] = 0xB2, 0x87
    w3, w2 = orc.synth_mxfp4(I, H, 11), orc.synth_mxfp4(H, I, 12)
    write_safetensors(tmp_path / "model.safetensors", [
        (p + "w1.weight_packed", "U8", [I, H], w1.tobytes()),
        (p + "w1.weight_scale", "U8", [I, H // 32], np.full(I * H // 32, 127, np.uint8).tobytes()),
        (p + "w3.weight_packed", "U8", [I, H], w3.data.tobytes()),
        (p + "w3.weight_scale", "U8", [I, H // 32], w3.scale.tobytes()),
        (p + "w2.weight_packed", "U8", [H, I], w2.data.tobytes()),
        (p + "w2.weight_scale", "U8", [H, I // 32], w2.scale.tobytes())])
    ctx.pool_load_mxfp4(R.Shards(str(tmp_path)), R.NAMING_KIMI_K3_MXFP4, layer, [0], H, I)
    slot = ctx.pool_get(layer, 0)
    assert slot is not None
    gate = C.cast(slot, C.POINTER(A.RbtExpertSlot)).contents.gate
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    ctx.check(ctx.lib.rbt_dequant_rows_d(ctx.h, C.byref(gate), 0, 1, out.data_ptr()))
    ctx.sync()
    row = out.cpu().numpy()
    assert bits_equal(row[:4], np.array([1.0, -1.5, 6.0, -0.0], np.float32))
    assert np.all(row[4:] == 0)


def test_shape_and_name_errors_leave_no_partial_expert(ctx, orc, tmp_path):
    import rabbit_amd as R
    H, I, layer = 64, 32, 11
    good = [orc.synth_mxfp4(I, H, 1), orc.synth_mxfp4(I, H, 2), orc.synth_mxfp4(H, I, 3)]
    tensors = []
    for e in range(3):
        for name, q in zip(_qwen_names(layer, e), good):
            scale = q.scale.tobytes()
            if e == 2 and name.endswith("down_proj"):
                scale = scale[:-1]  # one byte short
            tensors += [(name + ".weight", "U8", [q.rows, q.cols // 2], q.data.tobytes()),
                        (name + ".weight_scale", "U8", [q.rows, q.cols // 32], scale)]
    write_safetensors(tmp_path / "model.safetensors", tensors)
    sh = R.Shards(str(tmp_path))
    with pytest.raises(R.RbtError) as ei:
        ctx.pool_load_mxfp4(sh, R.NAMING_QWEN38_MXFP4, layer, [0, 1, 2], H, I)
    assert ei.value.status == -2
    assert f"model.layers.{layer}.mlp.experts.2.down_proj.weight_scale" in str(ei.value)
    assert ctx.pool_get(layer, 0) is not None and ctx.pool_get(layer, 1) is not None
    assert ctx.pool_get(layer, 2) is None
    with pytest.raises(R.RbtError) as ei:
        ctx.pool_load_mxfp4(sh, R.NAMING_QWEN38_MXFP4, layer, [5], H, I)
    assert ei.value.status == -7 and "experts.5.gate_proj.weight" in str(ei.value)
    with pytest.raises(R.RbtError) as ei:
        ctx.pool_load_mxfp4(sh, R.NAMING_KIMI_K3_MXFP4, layer, [0], H, I)
    assert ei.value.status == -7 and "weight_packed" in str(ei.value)


def test_real_shape_checkpoint_load_rate_and_parity(ctx, orc, tmp_path):
    """Ten C1-shaped experts (267 MB) through the loader: the load rate is printed, the layer output
    checked against the oracle for one token."""
    import rabbit_amd as R
    H, I, E, k, layer = 8192, 2048, 10, 10, 20
    experts = _write_qwen_checkpoint(tmp_path, orc, layer, E, H, I, seed=900, nshards=3)
    sh = R.Shards(str(tmp_path))
    t0 = time.perf_counter()
    ctx.pool_load_mxfp4(sh, R.NAMING_QWEN38_MXFP4, layer, range(E), H, I)
    dt = time.perf_counter() - t0
    nbytes = E * 3 * (2048 * 8192 // 2 + 2048 * 8192 // 32)
    print(f"loaded {nbytes / 1e6:.1f} MB in {dt * 1e3:.1f} ms: {nbytes / dt / 1e9:.2f} GB/s (page cache -> HBM)")
    router = normal((E, H), 5, 0.05)
    ctx.moe_layer_set(layer, R.FAMILY_QWEN38, H, I, E, k, router)
    L = orc.MoeLayer(orc.FAMILY_QWEN38, H, I, E, k, router, experts)
    x = normal((1, H), 6)
    exp, eids, _ = L.forward(x, 1)
    out = np.empty(H, np.float32)
    ids = np.empty(k, np.int32)
    ctx.moe_forward(layer, x, 1, out, ids)
    assert np.array_equal(ids.reshape(1, k), eids)
    assert rel_l2(out, exp) < RTOL
