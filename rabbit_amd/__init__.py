"""rabbit_amd -- MI355X (gfx950) routed-expert dequant-matmul for ferrumox/rabbit.

Python front end over the C ABI (include/rabbit_amd.h, librabbit_amd.so), used by the tests and
the benchmark. Names and argument meaning follow the reference's Rust functions:

    kernels.rs   matmul, matmul_mxfp4, matmul_i4_grouped, matmul_qt      (y overwritten)
    quant.rs     QT::row_f32 (dequant_rows), QT::resident_bytes
    qwen38/moe.rs route (route_softmax_topk), glm52/moe.rs route (route_sigmoid_topk)
    glm52/moe.rs  unique_experts, apply_single_expert                    (out accumulated)
    expert_cache.rs ExpertCache::get / ensure_loaded  (pool_get / pool_put)
    qwen38/generate.rs moe_forward, glm52/moe.rs moe   (moe_forward; out overwritten)

Host numpy arrays go through the plain entry points (copied in and out per call, like the
reference's borrowed slices); torch device tensors go through the `_d` entry points on the
context's own HIP stream. Errors raise RbtError with the library's status and message; there is no
CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import abi
from .abi import (ACT_SILU, FAMILY_GLM52, FAMILY_KIMI_K3, FAMILY_QWEN38, QT_F32, QT_I4_GROUPED, QT_MXFP4,
                  RbtExpertSlot, RbtMoeLayerDesc, RbtQT)

__all__ = ["Context", "QT", "Slot", "Shards", "RbtError", "load", "QT_F32", "QT_I4_GROUPED", "QT_MXFP4",
           "FAMILY_QWEN38", "FAMILY_GLM52", "FAMILY_KIMI_K3", "ACT_SILU", "NAMING_QWEN38_MXFP4",
           "NAMING_KIMI_K3_MXFP4", "ACT_SITU", "situ"]
from .abi import NAMING_KIMI_K3_MXFP4, NAMING_QWEN38_MXFP4, ACT_SITU  # noqa: E402


def situ(beta, linear_beta=None):
    """Activation::Situ { beta, linear_beta } (glm52/moe.rs:49-52) for apply_single_expert / latent_moe."""
    return abi.RbtActivation(ACT_SITU, beta, 0.0 if linear_beta is None else linear_beta, int(linear_beta is not None))


class RbtError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{abi.STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


def load():
    return abi.load()


def _is_torch(a) -> bool:
    return hasattr(a, "data_ptr") and hasattr(a, "is_cuda")


def _ptr(a):
    if a is None:
        return None
    if _is_torch(a):
        if not a.is_cuda:
            raise ValueError("torch tensors passed to rabbit_amd must live on the GPU")
        if not a.is_contiguous():
            raise ValueError("tensor must be contiguous")
        return a.data_ptr()
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("array must be C-contiguous")
        return a.ctypes.data
    if isinstance(a, int):
        return a
    raise TypeError(f"unsupported buffer {type(a)}")


class QT:
    """One quantized matrix (mirrors QT / QTKind, quant.rs:77-110). data/scale are numpy arrays
    (host) or torch GPU tensors (device)."""

    def __init__(self, kind, rows, cols, data, scale=None, group_size=0):
        self.kind, self.rows, self.cols = kind, rows, cols
        self.data, self.scale, self.group_size = data, scale, group_size

    @staticmethod
    def mxfp4(data, scale, rows, cols):
        return QT(QT_MXFP4, rows, cols, data, scale, 32)

    @staticmethod
    def i4g(data, scale, rows, cols, gs):
        return QT(QT_I4_GROUPED, rows, cols, data, scale, gs)

    @staticmethod
    def f32(w, rows, cols):
        return QT(QT_F32, rows, cols, w)

    @property
    def on_device(self) -> bool:
        return _is_torch(self.data)

    def c(self) -> RbtQT:
        return RbtQT(self.rows, self.cols, self.kind, _ptr(self.data), _ptr(self.scale), self.group_size)

    def resident_bytes(self) -> int:
        q = self.c()
        return abi.load().rbt_qt_resident_bytes(C.byref(q))


class Shards:
    """The safetensors shards of a checkpoint directory (Shards::open, safetensors.rs:230-349); host
    only, no GPU needed."""

    def __init__(self, directory: str):
        self.lib = abi.load()
        h = C.c_void_p()
        st = self.lib.rbt_shards_open(directory.encode(), C.byref(h))
        if st != 0:
            raise RbtError(st, self.lib.rbt_shards_last_error().decode())
        self.h = h

    def _check(self, st):
        if st != 0:
            raise RbtError(st, self.lib.rbt_shards_last_error().decode())

    def __len__(self):
        return self.lib.rbt_shards_count(self.h)

    def find(self, name: str) -> dict:
        ti = abi.RbtTensorInfo()
        self._check(self.lib.rbt_shards_find(self.h, name.encode(), C.byref(ti)))
        return {"file_index": ti.file_index, "offset": ti.offset, "nbytes": ti.nbytes,
                "dtype": ti.dtype.decode(), "shape": [ti.shape[i] for i in range(ti.ndim)]}

    def read(self, name: str) -> np.ndarray:
        n = self.find(name)["nbytes"]
        out = np.empty(max(n, 1), np.uint8)
        self._check(self.lib.rbt_shards_read(self.h, name.encode(), out.ctypes.data, out.size))
        return out[:n]

    def read_range(self, name: str, offset: int, n: int) -> np.ndarray:
        out = np.empty(max(n, 1), np.uint8)
        self._check(self.lib.rbt_shards_read_range(self.h, name.encode(), offset, out.ctypes.data, n))
        return out[:n]

    def close(self):
        if getattr(self, "h", None):
            self.lib.rbt_shards_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Slot:
    """One expert (mirrors ExpertSlot / GateUp, expert_cache.rs:640-650)."""

    def __init__(self, eid, down: QT, gate: QT | None = None, up: QT | None = None, gate_up: QT | None = None):
        self.eid, self.down, self.gate, self.up, self.gate_up = eid, down, gate, up, gate_up

    def c(self) -> RbtExpertSlot:
        z = RbtQT()
        return RbtExpertSlot(self.eid, int(self.gate_up is not None), self.gate.c() if self.gate else z,
                             self.up.c() if self.up else z, self.gate_up.c() if self.gate_up else z, self.down.c())


class Context:
    """An rbt_ctx on one HIP device: stream, scratch, HBM-resident expert pool, MoE layers."""

    def __init__(self, device: int = 0):
        self.lib = abi.load()
        h = C.c_void_p()
        rc = self.lib.rbt_init(C.byref(h), device)
        if rc != 0:
            raise RbtError(rc, (self.lib.rbt_last_error(None) or b"rbt_init failed").decode())
        self.h = h
        self._keep = []  # host arrays referenced by device-layer descriptors

    # -- plumbing ---------------------------------------------------------------------------
    def close(self):
        if self.h:
            self.lib.rbt_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc: int):
        if rc != 0:
            raise RbtError(rc, (self.lib.rbt_last_error(self.h) or b"").decode())
        return rc

    def sync(self):
        self.check(self.lib.rbt_sync(self.h))

    @property
    def stream(self) -> int:
        return self.lib.rbt_stream(self.h) or 0

    def torch_stream(self):
        """The context's stream as a torch ExternalStream (for HIP events / interop)."""
        import torch
        return torch.cuda.ExternalStream(self.stream)

    @staticmethod
    def _torch_sync():
        import torch
        torch.cuda.synchronize()

    # -- quant.rs ---------------------------------------------------------------------------
    def dequant_rows(self, w: QT, row0: int, nrows: int, out=None):
        q = w.c()
        if w.on_device:
            import torch
            if out is None:
                out = torch.empty(nrows * w.cols, dtype=torch.float32, device=w.data.device)
            self._torch_sync()
            self.check(self.lib.rbt_dequant_rows_d(self.h, C.byref(q), row0, nrows, _ptr(out)))
            self.sync()
            return out
        if out is None:
            out = np.empty(nrows * w.cols, np.float32)
        self.check(self.lib.rbt_dequant_rows(self.h, C.byref(q), row0, nrows, _ptr(out)))
        return out

    # -- kernels.rs -------------------------------------------------------------------------
    def matmul_qt(self, y, x, w: QT, s: int):
        q = w.c()
        if _is_torch(x):
            self._torch_sync()
            self.check(self.lib.rbt_matmul_qt_d(self.h, _ptr(y), _ptr(x), C.byref(q), s))
            self.sync()
        else:
            self.check(self.lib.rbt_matmul_qt(self.h, _ptr(y), _ptr(x), C.byref(q), s))
        return y

    def matmul(self, y, x, w, s, i, o):
        return self.matmul_qt(y, x, QT.f32(w, o, i), s)

    def matmul_mxfp4(self, y, x, data, block_scale, s, i, o):
        return self.matmul_qt(y, x, QT.mxfp4(data, block_scale, o, i), s)

    def matmul_i4_grouped(self, y, x, q4, scale, group_size, s, i, o):
        return self.matmul_qt(y, x, QT.i4g(q4, scale, o, i, group_size), s)

    # -- routers ----------------------------------------------------------------------------
    def route_softmax_topk(self, logits, s, n, k, ids, w):
        if _is_torch(logits):
            self._torch_sync()
            self.check(self.lib.rbt_route_softmax_topk_d(self.h, _ptr(logits), s, n, k, _ptr(ids), _ptr(w)))
            self.sync()
        else:
            self.check(self.lib.rbt_route_softmax_topk(self.h, _ptr(logits), s, n, k, _ptr(ids), _ptr(w)))
        return ids, w

    def route_sigmoid_topk(self, logits, bias, s, n, k, norm_topk, routed_scale, ids, w, n_group=1, topk_group=1):
        args = (self.h, _ptr(logits), _ptr(bias), s, n, k, int(norm_topk), float(routed_scale), n_group,
                topk_group, _ptr(ids), _ptr(w))
        if _is_torch(logits):
            self._torch_sync()
            self.check(self.lib.rbt_route_sigmoid_topk_d(*args))
            self.sync()
        else:
            self.check(self.lib.rbt_route_sigmoid_topk(*args))
        return ids, w

    def unique_experts(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        s, k = ids.shape
        out = np.zeros(max(1, s * k), np.int32)
        n = self.lib.rbt_unique_experts(_ptr(ids), s, k, _ptr(out))
        if n < 0:
            raise RbtError(n, "rbt_unique_experts")
        return out[:n]

    # -- experts ----------------------------------------------------------------------------
    def apply_single_expert(self, slot, ids, w, s, k, x, d, i, out, activation=ACT_SILU):
        """slot: a Slot (host or device weights) or a pool pointer from pool_get(). activation: ACT_SILU
        or an abi.RbtActivation (situ(beta, linear_beta))."""
        if isinstance(slot, C._Pointer):
            sc = slot
        elif isinstance(slot, (int, C.c_void_p)):
            sc = C.cast(slot, C.POINTER(RbtExpertSlot))
        else:
            sc = C.pointer(slot.c())
        par = isinstance(activation, abi.RbtActivation)
        dev = _is_torch(x)
        if dev:
            self._torch_sync()
        if par:
            fn = self.lib.rbt_apply_single_expert_act_d if dev else self.lib.rbt_apply_single_expert_act
            self.check(fn(self.h, sc, _ptr(ids), _ptr(w), s, k, _ptr(x), d, i, C.byref(activation), _ptr(out)))
        else:
            fn = self.lib.rbt_apply_single_expert_d if dev else self.lib.rbt_apply_single_expert
            self.check(fn(self.h, sc, _ptr(ids), _ptr(w), s, k, _ptr(x), d, i, activation, _ptr(out)))
        if dev:
            self.sync()
        return out

    def latent_moe(self, layer, moe_hidden, down_proj: QT, up_proj: QT, x, s, out, norm=None, eps=1e-5,
                   activation=None, ids_out=None, w_out=None, sync=True):
        """K3's latent MoE (kimi_k3/moe.rs:64-116) on device buffers: route with `layer`'s router at
        full width, its experts (pool, shaped for moe_hidden) on down_proj(x), optional rmsnorm, then
        up_proj. out [s, hidden] is overwritten."""
        act = activation if activation is not None else abi.RbtActivation(ACT_SILU, 0.0, 0.0, 0)
        lw = abi.RbtLatentMoeDesc(moe_hidden, down_proj.c(), up_proj.c(), _ptr(norm), eps, act)
        if sync:
            self._torch_sync()
        self.check(self.lib.rbt_latent_moe_d(self.h, layer, C.byref(lw), _ptr(x), s, _ptr(out), _ptr(ids_out),
                                             _ptr(w_out)))
        if sync:
            self.sync()
        return out

    # -- pool (ExpertCache) -----------------------------------------------------------------
    def pool_put(self, layer: int, slot: Slot):
        sc = slot.c()
        if slot.down.on_device:
            self.check(self.lib.rbt_pool_put_device(self.h, layer, C.byref(sc)))
        else:
            self.check(self.lib.rbt_pool_put(self.h, layer, C.byref(sc)))

    def pool_alloc(self, layer, eid, kind, d, i, group_size=32):
        p = self.lib.rbt_pool_alloc(self.h, layer, eid, kind, d, i, group_size)
        if not p:
            raise RbtError(-5, (self.lib.rbt_last_error(self.h) or b"").decode())
        return p

    def pool_get(self, layer, eid):
        p = self.lib.rbt_pool_get(self.h, layer, eid)
        return p if p else None

    def pool_resident_bytes(self) -> int:
        return self.lib.rbt_pool_resident_bytes(self.h)

    def synth_mxfp4(self, data_ptr, scale_ptr, rows, cols, seed, exp_lo=119, exp_hi=123):
        self.check(self.lib.rbt_synth_mxfp4_d(self.h, data_ptr, scale_ptr, rows, cols, seed, exp_lo, exp_hi))

    def synth_i4g(self, data_ptr, scale_ptr, rows, cols, gs, seed, s_lo=0.005, s_hi=0.02):
        self.check(self.lib.rbt_synth_i4g_d(self.h, data_ptr, scale_ptr, rows, cols, gs, seed, s_lo, s_hi))

    # -- token mixers (device tensors) ------------------------------------------------------
    def gdn_step(self, n_v, n_k, d_k, d_v, conv_weight, a_log, dt_bias, norm_weight, eps, conv_state, states,
                 qkv_pre, z, a, b, out, kernel=4, sync=True):
        """rbt_gdn_step_d: one token through a GDN layer's conv + step_token (qwen38/gdn.rs:142);
        conv_state and states are updated in place."""
        d = abi.RbtGdnDesc(n_v, n_k, d_k, d_v, kernel, _ptr(conv_weight), _ptr(a_log), _ptr(dt_bias),
                           _ptr(norm_weight), eps)
        if sync:
            self._torch_sync()
        self.check(self.lib.rbt_gdn_step_d(self.h, C.byref(d), _ptr(conv_state), _ptr(states), _ptr(qkv_pre),
                                           _ptr(z), _ptr(a), _ptr(b), _ptr(out)))
        if sync:
            self.sync()
        return out

    def gqa_step(self, n_heads, n_kv, head_dim, rope_dim, theta, attn_scale, eps, q_norm, k_norm, k_cache, v_cache,
                 cap, pos, qg, k, v, out, sync=True):
        """rbt_gqa_step_d: one token of GQA attention at position pos (qwen38/generate.rs:226-255)."""
        d = abi.RbtGqaDesc(n_heads, n_kv, head_dim, rope_dim, theta, attn_scale, eps, _ptr(q_norm), _ptr(k_norm))
        if sync:
            self._torch_sync()
        self.check(self.lib.rbt_gqa_step_d(self.h, C.byref(d), _ptr(k_cache), _ptr(v_cache), cap, pos, _ptr(qg),
                                           _ptr(k), _ptr(v), _ptr(out)))
        if sync:
            self.sync()
        return out

    # -- instrumentation --------------------------------------------------------------------
    def profile_enable(self, on: bool = True):
        self.check(self.lib.rbt_profile_enable(self.h, int(on)))

    def profile_read(self, reset: bool = True) -> dict:
        p = abi.RbtProfile()
        self.check(self.lib.rbt_profile_read(self.h, C.byref(p), int(reset)))
        return {f: getattr(p, f) for f, _ in abi.RbtProfile._fields_}

    def profile_kernels(self, on: bool = True):
        """Per-kernel timing: every launch records events at its own start and end."""
        self.check(self.lib.rbt_profile_kernels(self.h, int(on)))

    def profile_kernels_read(self, reset: bool = True) -> dict:
        """{kernel name: (launches, mean microseconds)} of the launches recorded so far."""
        cap = 64
        buf = (abi.RbtKernelStat * cap)()
        n = C.c_size_t()
        self.check(self.lib.rbt_profile_kernels_read(self.h, buf, cap, C.byref(n), int(reset)))
        out = {}
        for i in range(min(n.value, cap)):
            s = buf[i]
            if s.launches:
                out[s.name.decode(errors="replace")] = (int(s.launches), 1e3 * s.total_ms / s.launches)
        return out

    # -- MoE layer ----------------------------------------------------------------------------
    def moe_layer_set(self, layer, family, hidden, moe_inter, n_experts, topk, router, shared: Slot | None = None,
                      shared_gate=None, router_bias=None, logit_bias=None, norm_topk=True, routed_scale=1.0,
                      n_group=1, topk_group=1):
        d = RbtMoeLayerDesc()
        d.family, d.hidden, d.moe_inter, d.n_experts, d.topk = family, hidden, moe_inter, n_experts, topk
        d.router, d.router_bias, d.logit_bias = _ptr(router), _ptr(router_bias), _ptr(logit_bias)
        d.norm_topk, d.routed_scale, d.n_group, d.topk_group = int(norm_topk), routed_scale, n_group, topk_group
        d.has_shared = int(shared is not None)
        if shared is not None:
            d.shared = shared.c()
        d.shared_gate = _ptr(shared_gate)
        if _is_torch(router):
            self._keep.append((router, shared, shared_gate, router_bias, logit_bias))
            self.check(self.lib.rbt_moe_layer_set_device(self.h, layer, C.byref(d)))
        else:
            self.check(self.lib.rbt_moe_layer_set(self.h, layer, C.byref(d)))

    def rmsnorm(self, v, w, s, n, eps, one_plus=False, sync=True):
        """rmsnorm (kimi_linear/ops.rs:46) or rmsnorm_1p (qwen38/ops.rs:25) of device rows v[s, n] in
        place."""
        if sync:
            self._torch_sync()
        fn = self.lib.rbt_rmsnorm_1p_d if one_plus else self.lib.rbt_rmsnorm_d
        self.check(fn(self.h, _ptr(v), _ptr(w), s, n, eps))
        if sync:
            self.sync()
        return v

    def pool_load_mxfp4(self, shards: Shards, naming, layer, eids, hidden, moe_inter):
        """ensure_loaded for MXFP4 experts read verbatim from safetensors shards (expert_cache.rs:
        1227-1256): the experts `eids` of `layer` into the HBM pool."""
        e = np.ascontiguousarray(np.asarray(eids, np.uint32))
        self.check(self.lib.rbt_pool_load_mxfp4(self.h, shards.h, naming, layer, e.ctypes.data, e.size, hidden,
                                                moe_inter))

    def moe_sublayer(self, layer, x, s, post_ln, eps, ids_out=None, w_out=None, sync=True):
        """x += moe_forward(rmsnorm_1p(x, post_ln)) in place (qwen38/generate.rs:397-413)."""
        if _is_torch(x):
            if sync:
                self._torch_sync()
            self.check(self.lib.rbt_moe_sublayer_d(self.h, layer, _ptr(x), s, _ptr(post_ln), eps, _ptr(ids_out),
                                                   _ptr(w_out)))
            if sync:
                self.sync()
        else:
            self.check(self.lib.rbt_moe_sublayer(self.h, layer, _ptr(x), s, _ptr(post_ln), eps, _ptr(ids_out),
                                                 _ptr(w_out)))
        return x

    def moe_forward_noalloc(self, layer, x, s, out, ids_out=None, w_out=None, sync=True):
        """rbt_moe_forward_noalloc_d: moe_forward on device tensors with every per-call buffer taken
        from the device's fixed scratch array (no allocation in the call)."""
        if sync:
            self._torch_sync()
        self.check(self.lib.rbt_moe_forward_noalloc_d(self.h, layer, _ptr(x), s, _ptr(out), _ptr(ids_out),
                                                      _ptr(w_out)))
        if sync:
            self.sync()
        return out

    def moe_forward(self, layer, x, s, out, ids_out=None, w_out=None, sync=True):
        if _is_torch(x):
            if sync:
                self._torch_sync()
            self.check(self.lib.rbt_moe_forward_d(self.h, layer, _ptr(x), s, _ptr(out), _ptr(ids_out),
                                                  _ptr(w_out)))
            if sync:
                self.sync()
        else:
            self.check(self.lib.rbt_moe_forward(self.h, layer, _ptr(x), s, _ptr(out), _ptr(ids_out), _ptr(w_out)))
        return out
