"""ctypes front end for the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it as
the checker / CPU baseline. The product (rabbit_amd) never imports it.

Every function takes and returns numpy arrays; the C restatement it wraps cites the reference
function it follows (oracle/rabbit_oracle.c).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

QT_F32, QT_I4_GROUPED, QT_MXFP4 = 0, 1, 2
FAMILY_QWEN38, FAMILY_GLM52, FAMILY_KIMI_K3 = 0, 1, 2


class OrcQT(C.Structure):
    _fields_ = [("rows", C.c_size_t), ("cols", C.c_size_t), ("kind", C.c_int),
                ("data", C.c_void_p), ("scale", C.c_void_p), ("group_size", C.c_size_t)]


class OrcSlot(C.Structure):
    _fields_ = [("eid", C.c_uint32), ("fused", C.c_int), ("gate", OrcQT), ("up", OrcQT),
                ("gate_up", OrcQT), ("down", OrcQT)]


class OrcMoeLayer(C.Structure):
    _fields_ = [("family", C.c_int), ("hidden", C.c_size_t), ("moe_inter", C.c_size_t),
                ("n_experts", C.c_size_t), ("topk", C.c_size_t), ("router", C.c_void_p),
                ("router_bias", C.c_void_p), ("logit_bias", C.c_void_p), ("norm_topk", C.c_int),
                ("routed_scale", C.c_float), ("n_group", C.c_size_t), ("topk_group", C.c_size_t),
                ("has_shared", C.c_int), ("shared", OrcSlot), ("shared_gate", C.c_void_p),
                ("experts", C.c_void_p)]


ACT_SILU, ACT_SITU = 0, 1


class OrcAct(C.Structure):
    _fields_ = [("kind", C.c_int), ("beta", C.c_float), ("linear_beta", C.c_float), ("has_linear_beta", C.c_int)]


def situ(beta, linear_beta=None) -> OrcAct:
    """Activation::Situ { beta, linear_beta } (glm52/moe.rs:49-52)."""
    return OrcAct(ACT_SITU, beta, 0.0 if linear_beta is None else linear_beta, int(linear_beta is not None))


class OrcLatent(C.Structure):
    _fields_ = [("moe_hidden", C.c_size_t), ("down_proj", OrcQT), ("up_proj", OrcQT), ("norm", C.c_void_p),
                ("eps", C.c_float), ("act", OrcAct)]


def build(force: bool = False) -> str:
    """Compile liboracle.so with oracle/Makefile (gcc, -ffp-contract=off)."""
    import subprocess
    if force and os.path.exists(_LIB_PATH):
        os.remove(_LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run oracle.build() or `make -C oracle`")
        L = C.CDLL(_LIB_PATH)
        P, S, F, I = C.c_void_p, C.c_size_t, C.c_float, C.c_int
        L.orc_e2m1_decode.restype = F
        L.orc_e2m1_decode.argtypes = [C.c_uint8]
        L.orc_e8m0_decode.restype = F
        L.orc_e8m0_decode.argtypes = [C.c_uint8]
        L.orc_row_f32.argtypes = [C.POINTER(OrcQT), S, P]
        L.orc_resident_bytes.restype = S
        L.orc_resident_bytes.argtypes = [C.POINTER(OrcQT)]
        L.orc_matmul.argtypes = [P, P, P, S, S, S]
        L.orc_matmul_mxfp4_scalar.argtypes = [P, P, P, P, S, S, S]
        L.orc_matmul_mxfp4_avx2.argtypes = [P, P, P, P, S, S, S]
        L.orc_matmul_mxfp4_avx512.argtypes = [P, P, P, P, S, S, S]
        L.orc_matmul_mxfp4.argtypes = [P, P, P, P, S, S, S]
        L.orc_matmul_mxfp4.restype = I
        L.orc_matmul_i4_grouped.argtypes = [P, P, P, P, S, S, S, S]
        L.orc_matmul_qt.argtypes = [P, P, C.POINTER(OrcQT), S, I]
        L.orc_cpu_has_avx512.restype = I
        L.orc_cpu_has_avx2.restype = I
        L.orc_set_threads.argtypes = [I]
        L.orc_get_threads.restype = I
        L.orc_route_softmax.restype = S
        L.orc_route_softmax.argtypes = [P, S, S, P, P]
        L.orc_route_sigmoid.restype = S
        L.orc_route_sigmoid.argtypes = [P, P, S, S, I, F, S, S, P, P]
        L.orc_unique_experts.restype = S
        L.orc_unique_experts.argtypes = [P, S, S, P]
        L.orc_siluf.restype = F
        L.orc_siluf.argtypes = [F]
        L.orc_sigmoid.restype = F
        L.orc_sigmoid.argtypes = [F]
        L.orc_apply_single_expert.argtypes = [C.POINTER(OrcSlot), P, P, S, S, P, S, S, I, P]
        L.orc_moe_forward.restype = I
        L.orc_moe_forward.argtypes = [C.POINTER(OrcMoeLayer), P, S, I, P, P, P]
        L.orc_router_logits.argtypes = [C.POINTER(OrcMoeLayer), P, S, P]
        L.orc_rmsnorm.argtypes = [P, P, S, F]
        L.orc_act_combine.restype = F
        L.orc_act_combine.argtypes = [C.POINTER(OrcAct), F, F]
        L.orc_apply_single_expert_act.argtypes = [C.POINTER(OrcSlot), P, P, S, S, P, S, S, I, C.POINTER(OrcAct), P]
        L.orc_moe_route.argtypes = [C.POINTER(OrcMoeLayer), P, S, P, P]
        L.orc_latent_moe.restype = I
        L.orc_latent_moe.argtypes = [C.POINTER(OrcMoeLayer), C.POINTER(OrcLatent), P, S, I, P, P, P]
        L.orc_rmsnorm_1p.argtypes = [P, P, S, F]
        L.orc_moe_sublayer.restype = I
        L.orc_moe_sublayer.argtypes = [C.POINTER(OrcMoeLayer), P, S, P, F, I, P, P]
        L.orc_short_conv_step.argtypes = [P, S, S, P, P, P]
        L.orc_gdn_alpha.restype = F
        L.orc_gdn_alpha.argtypes = [F, F, F]
        L.orc_kda_step.argtypes = [P, S, S, P, P, P, F, F, P]
        L.orc_gdn_prepare_qk.argtypes = [P, P, S]
        L.orc_gdn_output_gate.argtypes = [P, P, P, S, F]
        L.orc_gdn_step_token.restype = I
        L.orc_gdn_step_token.argtypes = [P, S, S, S, P, S, P, P, P, P, P, P, F, P]
        L.orc_rope_half.argtypes = [P, S, S, F]
        L.orc_gqa_attend.argtypes = [P, S, P, P, S, S, S, F, P]
        L.orc_gqa_step.restype = I
        L.orc_gqa_step.argtypes = [P, P, P, S, S, S, P, P, F, S, F, F, P, P, S, P]
        L.orc_synth_mix64.restype = C.c_uint64
        L.orc_synth_mix64.argtypes = [C.c_uint64]
        L.orc_synth_mxfp4.argtypes = [P, P, S, S, C.c_uint64, C.c_uint32, C.c_uint32]
        L.orc_synth_i4g.argtypes = [P, P, S, S, S, C.c_uint64, F, F]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return lib().orc_get_threads()


def e2m1_decode(n: int) -> float:
    return lib().orc_e2m1_decode(n)


def e8m0_decode(b: int) -> float:
    return lib().orc_e8m0_decode(b)


def e8m0_decode_bits(b: int) -> int:
    return int(np.array([e8m0_decode(b)], dtype=np.float32).view(np.uint32)[0])


# --- quantized matrices ------------------------------------------------------------------------
class QT:
    """Host copy of one quantized matrix (mirrors QT, quant.rs:77-110). Keeps its arrays alive."""

    def __init__(self, kind, rows, cols, data, scale=None, group_size=0):
        self.kind, self.rows, self.cols, self.group_size = kind, rows, cols, group_size
        self.data, self.scale = data, scale
        self.c = OrcQT(rows, cols, kind, _p(data), _p(scale), group_size)

    @staticmethod
    def mxfp4(data, scale, rows, cols):
        data, scale = _u8(data).reshape(-1), _u8(scale).reshape(-1)
        assert data.size == rows * ((cols + 1) // 2) and scale.size == rows * ((cols + 31) // 32)
        return QT(QT_MXFP4, rows, cols, data, scale)

    @staticmethod
    def i4g(data, scale, rows, cols, gs):
        data, scale = _u8(data).reshape(-1), _f32(scale).reshape(-1)
        assert data.size == rows * ((cols + 1) // 2) and scale.size == rows * ((cols + gs - 1) // gs)
        return QT(QT_I4_GROUPED, rows, cols, data, scale, gs)

    @staticmethod
    def f32(w, rows, cols):
        w = _f32(w).reshape(-1)
        assert w.size == rows * cols
        return QT(QT_F32, rows, cols, w)

    def row_f32(self, r: int) -> np.ndarray:
        out = np.empty(self.cols, np.float32)
        lib().orc_row_f32(C.byref(self.c), r, _p(out))
        return out

    def dense(self) -> np.ndarray:
        return np.stack([self.row_f32(r) for r in range(self.rows)]) if self.rows else \
            np.zeros((0, self.cols), np.float32)

    def resident_bytes(self) -> int:
        return lib().orc_resident_bytes(C.byref(self.c))


def synth_mxfp4(rows, cols, seed, exp_lo=119, exp_hi=123) -> QT:
    data = np.empty(rows * ((cols + 1) // 2), np.uint8)
    scale = np.empty(rows * ((cols + 31) // 32), np.uint8)
    lib().orc_synth_mxfp4(_p(data), _p(scale), rows, cols, seed, exp_lo, exp_hi)
    return QT.mxfp4(data, scale, rows, cols)


def synth_i4g(rows, cols, gs, seed, s_lo=0.005, s_hi=0.02) -> QT:
    data = np.empty(rows * ((cols + 1) // 2), np.uint8)
    scale = np.empty(rows * ((cols + gs - 1) // gs), np.float32)
    lib().orc_synth_i4g(_p(data), _p(scale), rows, cols, gs, seed, s_lo, s_hi)
    return QT.i4g(data, scale, rows, cols, gs)


def mix64(z: int) -> int:
    return lib().orc_synth_mix64(z & (2**64 - 1))


# --- kernels -----------------------------------------------------------------------------------
def matmul(x, w, s, i, o):
    x, w = _f32(x), _f32(w)
    y = np.empty(s * o, np.float32)
    lib().orc_matmul(_p(y), _p(x), _p(w), s, i, o)
    return y


def matmul_mxfp4_scalar(x, data, scale, s, i, o):
    x, data, scale = _f32(x), _u8(data), _u8(scale)
    y = np.empty(s * o, np.float32)
    lib().orc_matmul_mxfp4_scalar(_p(y), _p(x), _p(data), _p(scale), s, i, o)
    return y


def matmul_mxfp4_tier(x, data, scale, s, i, o, tier="auto"):
    x, data, scale = _f32(x), _u8(data), _u8(scale)
    y = np.empty(s * o, np.float32)
    L = lib()
    fn = {"avx2": L.orc_matmul_mxfp4_avx2, "avx512": L.orc_matmul_mxfp4_avx512,
          "auto": L.orc_matmul_mxfp4}[tier]
    fn(_p(y), _p(x), _p(data), _p(scale), s, i, o)
    return y


def matmul_i4_grouped(x, q4, scale, gs, s, i, o):
    x, q4, scale = _f32(x), _u8(q4), _f32(scale)
    y = np.empty(s * o, np.float32)
    lib().orc_matmul_i4_grouped(_p(y), _p(x), _p(q4), _p(scale), gs, s, i, o)
    return y


def matmul_qt(x, w: QT, s, simd=False):
    x = _f32(x)
    y = np.empty(s * w.rows, np.float32)
    lib().orc_matmul_qt(_p(y), _p(x), C.byref(w.c), s, int(simd))
    return y


# --- routing -----------------------------------------------------------------------------------
def route_softmax(logits, k):
    logits = _f32(logits)
    n = logits.size
    ids = np.zeros(max(k, 1), np.int32)
    w = np.zeros(max(k, 1), np.float32)
    cnt = lib().orc_route_softmax(_p(logits), n, k, _p(ids), _p(w))
    return ids[:cnt].copy(), w[:cnt].copy()


def route_sigmoid(logits, k, bias=None, norm_topk=True, routed_scale=1.0, n_group=1, topk_group=1):
    logits = _f32(logits)
    n = logits.size
    b = None if bias is None else _f32(bias)
    ids = np.zeros(max(k, 1), np.int32)
    w = np.zeros(max(k, 1), np.float32)
    cnt = lib().orc_route_sigmoid(_p(logits), _p(b), n, k, int(norm_topk), routed_scale, n_group,
                                  topk_group, _p(ids), _p(w))
    return ids[:cnt].copy(), w[:cnt].copy()


def unique_experts(ids):
    ids = np.ascontiguousarray(ids, np.int32)
    s, k = ids.shape
    out = np.zeros(max(s * k, 1), np.int32)
    n = lib().orc_unique_experts(_p(ids), s, k, _p(out))
    return out[:n].copy()


def siluf(x: float) -> float:
    return lib().orc_siluf(x)


def sigmoid(x: float) -> float:
    return lib().orc_sigmoid(x)


def rmsnorm(v, w, eps):
    """kimi_linear/ops.rs:46-53 on each row of v (a copy)."""
    v = np.array(v, dtype=np.float32, copy=True)
    w = _f32(w)
    rows = v.reshape(-1, w.size)
    for r in range(rows.shape[0]):
        row = np.ascontiguousarray(rows[r])
        lib().orc_rmsnorm(_p(row), _p(w), w.size, eps)
        rows[r] = row
    return rows.reshape(v.shape)


def rmsnorm_1p(v, w, eps):
    """qwen38/ops.rs:25-33 on each row of v (a copy)."""
    v = np.array(v, dtype=np.float32, copy=True)
    w = _f32(w)
    rows = v.reshape(-1, w.size)
    for r in range(rows.shape[0]):
        row = np.ascontiguousarray(rows[r])
        lib().orc_rmsnorm_1p(_p(row), _p(w), w.size, eps)
        rows[r] = row
    return rows.reshape(v.shape)


# --- Qwen 3.8 token mixers (rabbit_oracle_mixers.c) ------------------------------------------
class GdnState:
    """One GDN layer's carried state: the short conv's history [conv_dim, kernel - 1] and the
    per-V-head delta-rule matrices [n_v, d_k, d_v] (kimi_linear/short_conv.rs:17-27,
    kimi_linear/kda.rs:92-101), all zero at the start."""

    def __init__(self, n_v, n_k, d_k, d_v, kernel=4):
        self.n_v, self.n_k, self.d_k, self.d_v, self.kernel = n_v, n_k, d_k, d_v, kernel
        self.key_dim, self.value_dim = n_k * d_k, n_v * d_v
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.conv = np.zeros(self.conv_dim * (kernel - 1), np.float32)
        self.heads = np.zeros(n_v * d_k * d_v, np.float32)


def short_conv_step(state: GdnState, x, weight):
    """kimi_linear/short_conv.rs:58-85 (updates state.conv); returns the conv output row."""
    x, weight = _f32(x), _f32(weight)
    out = np.empty(state.conv_dim, np.float32)
    lib().orc_short_conv_step(_p(state.conv), state.conv_dim, state.kernel, _p(x), _p(weight), _p(out))
    return out


def gdn_alpha(a_log, a, dt_bias) -> float:
    return lib().orc_gdn_alpha(a_log, a, dt_bias)


def gdn_prepare_qk(q, k):
    q, k = np.array(q, np.float32, copy=True), np.array(k, np.float32, copy=True)
    lib().orc_gdn_prepare_qk(_p(q), _p(k), q.size)
    return q, k


def gdn_output_gate(o, norm_weight, z, eps):
    o = np.array(o, np.float32, copy=True)
    nw, z = _f32(norm_weight), _f32(z)
    lib().orc_gdn_output_gate(_p(o), _p(nw), _p(z), o.size, eps)
    return o


def kda_step(s, q, k, v, alpha, beta):
    """kimi_linear/kda.rs:132-166 for one head; s [d_k, d_v] is updated in place. Returns o."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    assert s.dtype == np.float32 and s.flags["C_CONTIGUOUS"]
    o = np.empty(v.size, np.float32)
    lib().orc_kda_step(_p(s), q.size, v.size, _p(q), _p(k), _p(v), alpha, beta, _p(o))
    return o


def gdn_step_token(state: GdnState, qkv, z, a, b, a_log, dt_bias, norm_weight, eps):
    """qwen38/gdn.rs:142-196 (state.heads updated; qkv is the post-convolution row, not modified)."""
    qkv = np.array(qkv, dtype=np.float32, copy=True)
    z, a, b, a_log, dt_bias, nw = (_f32(v) for v in (z, a, b, a_log, dt_bias, norm_weight))
    out = np.empty(state.value_dim, np.float32)
    rc = lib().orc_gdn_step_token(_p(state.heads), state.n_v, state.d_k, state.d_v, _p(qkv), state.key_dim,
                                  _p(z), _p(a), _p(b), _p(a_log), _p(dt_bias), _p(nw), eps, _p(out))
    if rc:
        raise ValueError("bad GDN shape")
    return out


def gdn_step(state: GdnState, qkv_pre, conv_weight, z, a, b, a_log, dt_bias, norm_weight, eps):
    """qwen38/generate.rs:196-219 between the projections: the short conv, then step_token."""
    return gdn_step_token(state, short_conv_step(state, qkv_pre, conv_weight), z, a, b, a_log, dt_bias,
                          norm_weight, eps)


def rope_half(v, rope_dim, pos, theta):
    v = np.array(v, dtype=np.float32, copy=True)
    lib().orc_rope_half(_p(v), rope_dim, pos, theta)
    return v


def gqa_attend(q, k_cache, v_cache, n_kv, head_dim, scale):
    """qwen38/attention.rs:190-217; k_cache / v_cache [positions, n_kv * head_dim]."""
    q, kc, vc = _f32(q), _f32(k_cache), _f32(v_cache)
    positions = kc.size // (n_kv * head_dim)
    out = np.empty(q.size, np.float32)
    lib().orc_gqa_attend(_p(q), q.size // head_dim, _p(kc), _p(vc), positions, n_kv, head_dim, scale, _p(out))
    return out


class KvCache:
    """qwen38/attention.rs:54-82: K and V rows [cap, n_kv * head_dim], positions appended in order."""

    def __init__(self, n_kv, head_dim, cap):
        self.n_kv, self.head_dim, self.cap, self.len = n_kv, head_dim, cap, 0
        self.k = np.zeros((cap, n_kv * head_dim), np.float32)
        self.v = np.zeros((cap, n_kv * head_dim), np.float32)


def gqa_step(kv: KvCache, qg, k, v, n_heads, q_norm, k_norm, eps, rope_dim, theta, attn_scale):
    """qwen38/generate.rs:226-255 between the projections, at position kv.len (appends to kv)."""
    qg, k, v, qn, kn = (_f32(a) for a in (qg, k, v, q_norm, k_norm))
    assert kv.len < kv.cap
    ctx = np.empty(n_heads * kv.head_dim, np.float32)
    rc = lib().orc_gqa_step(_p(qg), _p(k), _p(v), n_heads, kv.n_kv, kv.head_dim, _p(qn), _p(kn), eps, rope_dim,
                            theta, attn_scale, _p(kv.k), _p(kv.v), kv.len, _p(ctx))
    if rc:
        raise ValueError("bad GQA shape")
    kv.len += 1
    return ctx


# --- experts and layers ------------------------------------------------------------------------
class Slot:
    """Host expert slot (mirrors ExpertSlot/GateUp). gate/up/gate_up/down are QT."""

    def __init__(self, eid, down, gate=None, up=None, gate_up=None):
        self.eid, self.gate, self.up, self.gate_up, self.down = eid, gate, up, gate_up, down
        empty = OrcQT()
        self.c = OrcSlot(eid, int(gate_up is not None), gate.c if gate else empty, up.c if up else empty,
                         gate_up.c if gate_up else empty, down.c)


def act_combine(act: OrcAct | None, g: float, u: float) -> float:
    """Activation::combine (glm52/moe.rs:58-70)."""
    return lib().orc_act_combine(C.byref(act) if act is not None else None, g, u)


def apply_single_expert(slot: Slot, ids, wts, x, d, i, out, simd=False, act: OrcAct | None = None):
    ids = np.ascontiguousarray(ids, np.int32)
    wts = _f32(wts)
    s, k = ids.shape
    x = _f32(x)
    assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    lib().orc_apply_single_expert_act(C.byref(slot.c), _p(ids), _p(wts), s, k, _p(x), d, i, int(simd),
                                      C.byref(act) if act is not None else None, _p(out))
    return out


class MoeLayer:
    """Host MoE layer (router + shared expert + routed experts)."""

    def __init__(self, family, hidden, moe_inter, n_experts, topk, router, experts, shared=None,
                 shared_gate=None, router_bias=None, logit_bias=None, norm_topk=True, routed_scale=1.0,
                 n_group=1, topk_group=1):
        self.router = _f32(router).reshape(-1)
        self.shared_gate = None if shared_gate is None else _f32(shared_gate)
        self.router_bias = None if router_bias is None else _f32(router_bias)
        self.logit_bias = None if logit_bias is None else _f32(logit_bias)
        self.experts = experts  # dict eid -> Slot (or list)
        self.shared = shared
        self.hidden, self.n_experts, self.topk = hidden, n_experts, topk
        ptrs = (C.POINTER(OrcSlot) * n_experts)()
        for e in range(n_experts):
            sl = experts.get(e) if isinstance(experts, dict) else experts[e]
            ptrs[e] = C.pointer(sl.c) if sl is not None else None
        self._ptrs = ptrs
        self.c = OrcMoeLayer(family, hidden, moe_inter, n_experts, topk, _p(self.router), _p(self.router_bias),
                             _p(self.logit_bias), int(norm_topk), routed_scale, n_group, topk_group,
                             int(shared is not None), shared.c if shared else OrcSlot(),
                             _p(self.shared_gate), C.cast(ptrs, C.c_void_p).value)

    def router_logits(self, x, s):
        x = _f32(x)
        out = np.empty(s * self.n_experts, np.float32)
        lib().orc_router_logits(C.byref(self.c), _p(x), s, _p(out))
        return out.reshape(s, self.n_experts)

    def forward(self, x, s, simd=False):
        x = _f32(x)
        out = np.empty(s * self.hidden, np.float32)
        k = min(self.topk, self.n_experts)
        ids = np.empty(max(s * k, 1), np.int32)
        w = np.empty(max(s * k, 1), np.float32)
        rc = lib().orc_moe_forward(C.byref(self.c), _p(x), s, int(simd), _p(out), _p(ids), _p(w))
        if rc != 0:
            raise RuntimeError("orc_moe_forward: routed expert missing from the pool")
        return out.reshape(s, self.hidden), ids[:s * k].reshape(s, k), w[:s * k].reshape(s, k)

    def route(self, x, s):
        """The layer's routing alone: ids, w [s, min(topk, E)]."""
        x = _f32(x)
        k = min(self.topk, self.n_experts)
        ids = np.empty(max(s * k, 1), np.int32)
        w = np.empty(max(s * k, 1), np.float32)
        lib().orc_moe_route(C.byref(self.c), _p(x), s, _p(ids), _p(w))
        return ids[:s * k].reshape(s, k), w[:s * k].reshape(s, k)

    def latent(self, x, s, moe_hidden, down_proj: QT, up_proj: QT, norm=None, eps=1e-5,
               act: OrcAct | None = None, simd=False):
        """K3's latent MoE (kimi_k3/moe.rs:64-116): this layer's router at full width, its experts at
        moe_hidden. Returns out [s, hidden], ids, w."""
        x = _f32(x)
        norm = None if norm is None else _f32(norm)
        lw = OrcLatent(moe_hidden, down_proj.c, up_proj.c, _p(norm), eps,
                       act if act is not None else OrcAct(ACT_SILU, 0.0, 0.0, 0))
        out = np.empty(s * up_proj.rows, np.float32)
        k = min(self.topk, self.n_experts)
        ids = np.empty(max(s * k, 1), np.int32)
        w = np.empty(max(s * k, 1), np.float32)
        rc = lib().orc_latent_moe(C.byref(self.c), C.byref(lw), _p(x), s, int(simd), _p(out), _p(ids), _p(w))
        if rc != 0:
            raise RuntimeError("orc_latent_moe: routed expert missing from the pool")
        return out.reshape(s, up_proj.rows), ids[:s * k].reshape(s, k), w[:s * k].reshape(s, k)

    def sublayer(self, x, s, post_ln, eps, simd=False):
        """x + moe_forward(rmsnorm_1p(x, post_ln)) (qwen38/generate.rs:397-413); returns a copy."""
        xo = np.array(_f32(x), copy=True)
        k = min(self.topk, self.n_experts)
        ids = np.empty(max(s * k, 1), np.int32)
        w = np.empty(max(s * k, 1), np.float32)
        post_ln = _f32(post_ln)
        rc = lib().orc_moe_sublayer(C.byref(self.c), _p(xo), s, _p(post_ln), eps, int(simd), _p(ids), _p(w))
        if rc != 0:
            raise RuntimeError("orc_moe_sublayer: routed expert missing from the pool")
        return xo.reshape(s, self.hidden), ids[:s * k].reshape(s, k), w[:s * k].reshape(s, k)
