"""Writes tests/golden/kats.json: the known-answer vectors of the reference's own tests for this
path, transcribed as data (inputs and expected outputs, each with the reference file:line it comes
from), plus the reference router test's HF transcription evaluated on its LCG logits.

Nothing here imports or runs the reference; the expected values are the literals its tests assert,
or (route_hf) the independent four-line algorithm its test compares against, evaluated in numpy.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def lcg_logits(n: int, seed: int) -> np.ndarray:
    """qwen38/moe.rs:105-113: u32 LCG, ((s >> 8) % 2000) as f32 / 100.0 - 10.0."""
    s = max(seed, 1) & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32((s >> 8) % 2000) / np.float32(100.0) - np.float32(10.0)
    return out


def hf_route(logits: np.ndarray, k: int):
    """The HF four-liner as transcribed at qwen38/moe.rs:89-103: softmax over all experts in f32,
    stable top-k by (prob desc, id asc), renormalise by the selected sum."""
    l = logits.astype(np.float32)
    mx = np.float32(l.max())
    exps = np.exp((l - mx).astype(np.float32)).astype(np.float32)
    total = np.float32(0.0)
    for v in exps:
        total = np.float32(total + v)
    probs = (exps / total).astype(np.float32)
    idx = sorted(range(len(probs)), key=lambda i: (-float(probs[i]), i))[:min(k, len(probs))]
    ssum = np.float32(0.0)
    for i in idx:
        ssum = np.float32(ssum + probs[i])
    return [int(i) for i in idx], [float(np.float32(probs[i] / ssum)) for i in idx]


def main():
    kats = {}
    kats["e2m1_table"] = {
        "ref": "quant.rs:858-866",
        "codes": list(range(16)),
        "values": [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    }
    kats["e8m0_points"] = {"ref": "quant.rs:887-893", "bytes": [127, 128, 126, 131], "values": [1.0, 2.0, 0.5, 16.0]}
    kats["disk_bytes"] = {
        "ref": "expert_cache.rs:1557-1566,1785-1787",
        "data": [0xB2, 0x87], "scale": [127], "cols": 4, "row0": [1.0, -1.5, 6.0, -0.0],
    }
    data = [4 | (4 << 4)] * 16 + [(7 | 8) | ((7 | 8) << 4)] * 4
    kats["mxfp4_two_block"] = {
        "ref": "kernels.rs:1388-1406", "cols": 40, "data": data, "block_scale": [127, 130],
        "x": [1.0] * 40, "y": [32.0 * 2.0 + 8.0 * -48.0],
    }
    vals = [1, -1, 2, 3, -2, 0]
    q = [0] * 3
    for i, v in enumerate(vals):
        q[i // 2] |= (v + 8) << (4 * (i % 2))
    kats["i4g_two_group"] = {
        "ref": "kernels.rs:1408-1428", "cols": 6, "gs": 3, "q4": q, "scale": [2.0, 5.0], "x": [1.0] * 6, "y": [9.0],
    }
    kats["matmul"] = {
        "ref": "kernels.rs:1323-1331", "s": 2, "i": 3, "o": 2,
        "x": [1.0, 2.0, 3.0, -1.0, 0.5, 2.0], "w": [1.0, 0.0, 0.0, 0.0, 1.0, 1.0], "y": [1.0, 5.0, -1.0, 2.5],
    }
    kats["route_select"] = {"ref": "qwen38/moe.rs:140-147", "logits": [0.0, 2.0, -1.0, 5.0, 0.5, -3.0, 1.0, 3.0],
                            "k": 3, "ids": [3, 7, 1]}
    kats["route_ties"] = {"ref": "qwen38/moe.rs:163-171",
                          "cases": [{"logits": [1.0, 1.0, 1.0, 1.0], "k": 2, "ids": [0, 1]},
                                    {"logits": [0.0, 5.0, 5.0, 5.0], "k": 2, "ids": [1, 2]}]}
    kats["route_k_ge_n"] = {"ref": "qwen38/moe.rs:173-182", "logits": [3.0, 1.0, 2.0], "k": 10, "ids": [0, 2, 1]}
    cases = []
    for seed in range(1, 6):
        l = lcg_logits(512, seed)
        ids, w = hf_route(l, 10)
        cases.append({"seed": seed, "ids": ids, "weights": w})
    kats["route_hf"] = {"ref": "qwen38/moe.rs:89-127", "n": 512, "k": 10, "tol": 1e-6, "cases": cases}
    kats["glm_select_vs_weight"] = {
        "ref": "glm52/moe.rs:920-943", "router": [10.0, 0.0, -10.0, 0.0], "bias": [0.0, 100.0], "x": [1.0, 0.0],
        "k": 1, "ids": [1], "weight": float(np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(10.0)))),
        "tol": 1e-5,
    }
    kats["glm_norm_topk"] = {"ref": "glm52/moe.rs:945-961", "routed_scale": 2.0, "tol": 1e-5}
    kats["glm_grouped"] = {
        "ref": "glm52/moe.rs:985-1006",
        "cases": [{"choice": [0.1, 0.2, 9.0, 8.0, 0.3, 0.4, 7.0, 6.5], "k": 3, "n_group": 4, "topk_group": 2,
                   "ids": [2, 3, 6]},
                  {"choice": [0.9] * 8, "k": 2, "n_group": 4, "topk_group": 1, "ids": [0, 1]}],
    }
    kats["fused_separate"] = {"ref": "glm52/moe.rs:592-626", "d": 6, "i": 8, "weights": [0.6, 1.3, -0.4]}
    kats["tier_cols"] = {"ref": "kernels.rs:1916-1983", "cols": [1, 7, 16, 17, 32, 33, 65], "rows": 3, "tol": 1e-4}
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats, f, indent=1)
    print("wrote", os.path.join(HERE, "kats.json"))


if __name__ == "__main__":
    main()
