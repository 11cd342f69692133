"""Host-side regeneration of the synthetic benchmark layers for the oracle (TEST INFRASTRUCTURE).

Rebuilds, byte for byte, the experts that rabbit_amd.workloads.build_layer generates on the device
(same counter-based generator and tensor seeds), but only those a given set of tokens routes to,
so the CPU oracle can run a full-size layer without materialising the whole pool.
"""
from __future__ import annotations

import numpy as np

from rabbit_amd.workloads import Config, router_weights, tensor_seed

from . import oracle as O


def host_qt(cfg: Config, rows, cols, seed):
    if cfg.kind == O.QT_MXFP4:
        return O.synth_mxfp4(rows, cols, seed, cfg.exp_lo, cfg.exp_hi)
    return O.synth_i4g(rows, cols, cfg.gs, seed, cfg.s_lo, cfg.s_hi)


def host_expert(cfg: Config, seed: int, eid: int) -> O.Slot:
    H, I = cfg.hidden, cfg.inter
    return O.Slot(eid, host_qt(cfg, H, I, tensor_seed(seed, eid, 2)),
                  gate=host_qt(cfg, I, H, tensor_seed(seed, eid, 0)),
                  up=host_qt(cfg, I, H, tensor_seed(seed, eid, 1)))


class HostLayer:
    """Router + shared expert on the host, routed experts generated on demand."""

    def __init__(self, cfg: Config, seed: int = 1000):
        self.cfg, self.seed = cfg, seed
        self.router, self.gate, self.logit_bias = router_weights(cfg, seed + 7)
        self.shared = host_expert(cfg, seed, cfg.n_experts) if cfg.shared else None
        self.experts: dict[int, O.Slot] = {}

    def _layer(self):
        c = self.cfg
        return O.MoeLayer(c.family, c.hidden, c.inter, c.n_experts, c.topk, self.router, self.experts,
                          shared=self.shared, shared_gate=self.gate, logit_bias=self.logit_bias, norm_topk=True,
                          routed_scale=1.0)

    def route(self, x: np.ndarray):
        """Oracle routing of tokens x [s, hidden] -> ids [s, k], weights [s, k]."""
        c = self.cfg
        s = x.shape[0]
        logits = self._layer().router_logits(x, s)
        k = min(c.topk, c.n_experts)
        ids = np.zeros((s, k), np.int32)
        w = np.zeros((s, k), np.float32)
        for t in range(s):
            if c.family == O.FAMILY_QWEN38:
                ids[t], w[t] = O.route_softmax(logits[t], k)
            else:
                ids[t], w[t] = O.route_sigmoid(logits[t], k, norm_topk=True, routed_scale=1.0)
        return ids, w

    def ensure(self, ids) -> None:
        for e in np.unique(np.asarray(ids)):
            if int(e) not in self.experts:
                self.experts[int(e)] = host_expert(self.cfg, self.seed, int(e))

    def forward(self, x: np.ndarray, simd: bool = False):
        ids, _ = self.route(x)
        self.ensure(ids)
        return self._layer().forward(x, x.shape[0], simd=simd)

    def sublayer(self, x: np.ndarray, post_ln: np.ndarray, eps: float, simd: bool = False):
        """x + moe_forward(rmsnorm_1p(x, post_ln)) (qwen38/generate.rs:397-413)."""
        ids, _ = self.route(O.rmsnorm_1p(x, post_ln, eps))
        self.ensure(ids)
        return self._layer().sublayer(x, x.shape[0], post_ln, eps, simd=simd)
