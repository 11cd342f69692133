"""Pins the fp64 truth (tests/f64_truth.py) that the per-token GPU parity checks fall back on.

* dense64 rounded to fp32 equals the oracle's row_f32 bit for bit over every E2M1 code byte and every
  E8M0 scale byte (0 -> 2^-127, 255 -> the +inf bits, quant.rs:353-396), and for grouped int4;
* layer64 agrees with the oracle's sequential-fp32 layer on small layers of both router families
  (softmax with a gated shared expert; sigmoid with norm_topk and an ungated shared expert) to the
  oracle's own rounding level, so a dropped term, a wrong sign or a swapped operand fails here.
"""
import numpy as np
import pytest

from f64_truth import dense64, layer64, rel_l2
from helpers import bits_equal


def test_dense64_mxfp4_every_code_and_scale(orc):
    rows, cols = 256, 512
    data = np.tile(np.arange(256, dtype=np.uint8), rows)              # every code byte in every row
    scale = np.repeat(np.arange(256, dtype=np.uint8), cols // 32)     # row r: scale byte r
    q = orc.QT.mxfp4(data, scale, rows, cols)
    got = dense64(q, "cpu").numpy().astype(np.float32)
    assert bits_equal(got, q.dense())


def test_dense64_i4g(orc):
    q = orc.synth_i4g(64, 96, 32, 7)
    got = dense64(q, "cpu").numpy().astype(np.float32)
    # one fp32 multiply in the reference: exact products of a 4-bit integer and an fp32 scale
    assert bits_equal(got, q.dense())


@pytest.mark.parametrize("family,kind,gated", [(0, 2, True), (1, 1, False), (2, 2, False)])
def test_layer64_matches_the_oracle_layer(orc, family, kind, gated):
    from rabbit_amd.workloads import Config
    from oracle.workload import HostLayer
    cfg = Config("tiny", family, 256, 128, 16, 4, kind, 3, gated_shared=gated, zipf_logit_bias=family == 2)
    host = HostLayer(cfg, 77)
    x = np.random.default_rng(5).standard_normal((3, 256)).astype(np.float32)
    exp, ids, _ = host.forward(x)
    truth = layer64(host, x, ids)
    for t in range(3):
        err = rel_l2(exp[t], truth[t])
        assert err < 2e-6, (t, err)


def test_check_token_rule_and_its_ceiling():
    """check_token: within 1e-5 of the oracle passes; farther passes only while the oracle is the
    one farther from the fp64 truth and the device stays within the 2e-5 ceiling."""
    from f64_truth import check_token
    rng = np.random.default_rng(3)
    truth = rng.standard_normal(4096)
    u = rng.standard_normal(4096)
    u /= np.linalg.norm(u) / np.linalg.norm(truth)  # |u| = |truth|: an offset c * u is c relative
    assert check_token(truth + 5e-6 * u, truth, truth)[3]                 # within 1e-5 of the oracle
    assert check_token(truth, truth + 1.5e-5 * u, truth)[3]               # the oracle is the one off
    assert not check_token(truth + 1.5e-5 * u, truth, truth)[3]           # the device is the one off
    # both 1.2e-5 from the truth on opposite sides: 2.4e-5 apart, over the ceiling
    assert not check_token(truth - 1.2e-5 * u, truth + 1.2e-5 * u, truth)[3]
    assert check_token(truth - 0.9e-5 * u, truth + 0.9e-5 * u, truth)[3]  # 1.8e-5 apart: under it
