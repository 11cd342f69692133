"""Synthetic workloads of the benchmark configurations (C0..C4), built in place in HBM.

Weights come from the library's counter-based generator (rbt_synth_*), so a host can regenerate
any expert byte for byte (oracle.synth_* uses the same formula). Activations and router weights
are seeded numpy normals uploaded once.

Seeds: expert e's gate/up/down use tensor seeds base + 4e + {0, 1, 2}; the shared expert uses
e = n_experts.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import FAMILY_GLM52, FAMILY_KIMI_K3, FAMILY_QWEN38, QT, QT_I4_GROUPED, QT_MXFP4, Slot


@dataclass
class Config:
    name: str
    family: int
    hidden: int
    inter: int
    n_experts: int
    topk: int
    kind: int
    tokens: int
    gs: int = 32
    shared: bool = True
    gated_shared: bool = False
    zipf_logit_bias: bool = False
    exp_lo: int = 119
    exp_hi: int = 123
    s_lo: float = 0.005
    s_hi: float = 0.02
    router_std: float = 0.02
    extra: dict = field(default_factory=dict)


CONFIGS = {
    "c0": Config("c0_single_expert", FAMILY_QWEN38, 8192, 2048, 1, 1, QT_MXFP4, 1, shared=False),
    "c1": Config("c1_qwen38_decode_b1", FAMILY_QWEN38, 8192, 2048, 512, 10, QT_MXFP4, 1, gated_shared=True),
    "c2": Config("c2_glm_i4g_decode_b1", FAMILY_GLM52, 6144, 2048, 256, 8, QT_I4_GROUPED, 1),
    "c3": Config("c3_k3_decode_b8_zipf", FAMILY_KIMI_K3, 7168, 2048, 384, 8, QT_MXFP4, 8, zipf_logit_bias=True),
    "c4": Config("c4_qwen38_prefill_512", FAMILY_QWEN38, 8192, 2048, 512, 10, QT_MXFP4, 512, gated_shared=True),
    # Kimi K3's routed MoE (kimi_k3/config.rs:245-275): 896 MXFP4 experts at moe_hidden 3584 with
    # moe_inter 3072, top-16 by sigmoid with a correction bias, Situ(4, 25), the routed-expert norm;
    # the latent projections as grouped int4 (group 32), the converter's --dense-bits 4 form
    "k3l": Config("k3_latent_decode_b1", FAMILY_KIMI_K3, 7168, 3072, 896, 16, QT_MXFP4, 1, shared=False,
                  extra={"moe_hidden": 3584, "proj_gs": 32, "situ": (4.0, 25.0), "latent_norm": True}),
}


def tensor_seed(base: int, eid: int, mat: int) -> int:
    return base + 4 * eid + mat


def expert_bytes(cfg: Config) -> int:
    """Resident bytes of one expert (gate + up + down)."""
    H, I = cfg.hidden, cfg.inter
    if cfg.kind == QT_MXFP4:
        per = lambda r, c: r * c // 2 + r * c // 32  # noqa: E731
    else:
        per = lambda r, c: r * c // 2 + r * (c // cfg.gs) * 4  # noqa: E731
    return 2 * per(I, H) + per(H, I)


def router_weights(cfg: Config, seed: int):
    rng = np.random.default_rng(seed)
    router = (rng.standard_normal((cfg.n_experts, cfg.hidden)) * cfg.router_std).astype(np.float32)
    gate = (rng.standard_normal(cfg.hidden) * 0.02).astype(np.float32) if cfg.gated_shared else None
    logit_bias = None
    if cfg.zipf_logit_bias:
        rank = rng.permutation(cfg.n_experts) + 1
        logit_bias = (2.0 * np.log(1.0 / rank)).astype(np.float32)
    return router, gate, logit_bias


def tokens(cfg: Config, n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((n, cfg.hidden)).astype(np.float32)


def _synth(ctx, kind, data_ptr, scale_ptr, rows, cols, seed, cfg):
    if kind == QT_MXFP4:
        ctx.synth_mxfp4(data_ptr, scale_ptr, rows, cols, seed, cfg.exp_lo, cfg.exp_hi)
    else:
        ctx.synth_i4g(data_ptr, scale_ptr, rows, cols, cfg.gs, seed, cfg.s_lo, cfg.s_hi)


def device_qt(ctx, cfg: Config, rows, cols, seed):
    import torch
    dev = torch.device("cuda")
    data = torch.empty(rows * cols // 2, dtype=torch.uint8, device=dev)
    if cfg.kind == QT_MXFP4:
        scale = torch.empty(rows * cols // 32, dtype=torch.uint8, device=dev)
        q = QT.mxfp4(data, scale, rows, cols)
    else:
        scale = torch.empty(rows * (cols // cfg.gs), dtype=torch.float32, device=dev)
        q = QT.i4g(data, scale, rows, cols, cfg.gs)
    _synth(ctx, cfg.kind, data.data_ptr(), scale.data_ptr(), rows, cols, seed, cfg)
    return q


def build_layer(ctx, cfg: Config, layer: int = 0, seed: int = 1000, n_resident: int | None = None):
    """Allocates and fills the layer's routed experts in the pool (HBM-resident), the shared expert
    and the router. Returns a dict with the host-side router arrays (for the oracle)."""
    import torch
    E = cfg.n_experts if n_resident is None else n_resident
    H, I = cfg.hidden, cfg.inter
    for e in range(E):
        p = ctx.pool_alloc(layer, e, cfg.kind, H, I, cfg.gs)
        s = p.contents
        for m, q in enumerate((s.gate, s.up, s.down)):
            _synth(ctx, cfg.kind, q.data, q.scale, q.rows, q.cols, tensor_seed(seed, e, m), cfg)
    router, gate, logit_bias = router_weights(cfg, seed + 7)
    shared = None
    if cfg.shared:
        shared = Slot(cfg.n_experts,
                      device_qt(ctx, cfg, H, I, tensor_seed(seed, cfg.n_experts, 2)),
                      gate=device_qt(ctx, cfg, I, H, tensor_seed(seed, cfg.n_experts, 0)),
                      up=device_qt(ctx, cfg, I, H, tensor_seed(seed, cfg.n_experts, 1)))
    dev = torch.device("cuda")
    t_router = torch.from_numpy(router).to(dev)
    t_gate = torch.from_numpy(gate).to(dev) if gate is not None else None
    t_lb = torch.from_numpy(logit_bias).to(dev) if logit_bias is not None else None
    ctx.sync()
    ctx.moe_layer_set(layer, cfg.family, H, I, cfg.n_experts, cfg.topk, t_router, shared=shared, shared_gate=t_gate,
                      logit_bias=t_lb, norm_topk=True, routed_scale=1.0)
    torch.cuda.synchronize()
    return {"router": router, "shared_gate": gate, "logit_bias": logit_bias, "shared": shared, "seed": seed}


def latent_host_params(cfg: Config, seed: int):
    """Router, correction bias and norm weight of the latent workload (host arrays)."""
    rng = np.random.default_rng(seed + 7)
    router = (rng.standard_normal((cfg.n_experts, cfg.hidden)) * cfg.router_std).astype(np.float32)
    bias = (rng.standard_normal(cfg.n_experts) * 0.01).astype(np.float32)
    norm = (1.0 + rng.standard_normal(cfg.extra["moe_hidden"]) * 0.1).astype(np.float32)
    return router, bias, norm


def build_latent_layer(ctx, cfg: Config, layer: int = 0, seed: int = 1000):
    """K3's latent MoE layer in HBM: routed experts at (moe_hidden, moe_inter) in the pool (tensor
    seeds as build_layer's), the router at full width, and the two projections (grouped int4,
    tensor seeds of eid n_experts and n_experts + 1). Returns the device pieces rbt_latent_moe_d
    takes."""
    import torch
    from . import situ
    MH, I, H, gs = cfg.extra["moe_hidden"], cfg.inter, cfg.hidden, cfg.extra["proj_gs"]
    for e in range(cfg.n_experts):
        p = ctx.pool_alloc(layer, e, cfg.kind, MH, I, cfg.gs)
        s = p.contents
        for m, q in enumerate((s.gate, s.up, s.down)):
            _synth(ctx, cfg.kind, q.data, q.scale, q.rows, q.cols, tensor_seed(seed, e, m), cfg)
    router, bias, norm = latent_host_params(cfg, seed)
    dev = torch.device("cuda")
    proj = []
    for j, (rows, cols) in enumerate(((MH, H), (H, MH))):
        data = torch.empty(rows * cols // 2, dtype=torch.uint8, device=dev)
        scale = torch.empty(rows * (cols // gs), dtype=torch.float32, device=dev)
        ctx.synth_i4g(data.data_ptr(), scale.data_ptr(), rows, cols, gs, tensor_seed(seed, cfg.n_experts + j, 0),
                      cfg.s_lo, cfg.s_hi)
        proj.append(QT.i4g(data, scale, rows, cols, gs))
    t_router = torch.from_numpy(router).to(dev)
    t_bias = torch.from_numpy(bias).to(dev)
    ctx.sync()
    ctx.moe_layer_set(layer, cfg.family, H, I, cfg.n_experts, cfg.topk, t_router, router_bias=t_bias,
                      norm_topk=True, routed_scale=1.0)
    torch.cuda.synchronize()
    beta, lb = cfg.extra["situ"]
    return {"down": proj[0], "up": proj[1], "norm": torch.from_numpy(norm).to(dev) if cfg.extra["latent_norm"]
            else None, "act": situ(beta, lb), "router": t_router, "bias": t_bias}
