"""ctypes declarations of the C ABI in include/rabbit_amd.h (librabbit_amd.so).

The library is the product: loading fails loudly when it is missing or was built without a symbol;
there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librabbit_amd.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "rabbit_amd.h")

RBT_OK = 0
RBT_E_INVALID = -1
RBT_E_SHAPE = -2
RBT_E_HIP = -3
RBT_E_NOT_RESIDENT = -4
RBT_E_NOMEM = -5
RBT_E_UNSUPPORTED = -6
STATUS_NAMES = {0: "RBT_OK", -1: "RBT_E_INVALID", -2: "RBT_E_SHAPE", -3: "RBT_E_HIP",
                -4: "RBT_E_NOT_RESIDENT", -5: "RBT_E_NOMEM", -6: "RBT_E_UNSUPPORTED", -7: "RBT_E_NOT_FOUND",
                -8: "RBT_E_FORMAT", -9: "RBT_E_IO"}

QT_F32, QT_I4_GROUPED, QT_MXFP4 = 0, 1, 2
FAMILY_QWEN38, FAMILY_GLM52, FAMILY_KIMI_K3 = 0, 1, 2
ACT_SILU, ACT_SITU = 0, 1


class RbtQT(C.Structure):
    _fields_ = [("rows", C.c_size_t), ("cols", C.c_size_t), ("kind", C.c_int32),
                ("data", C.c_void_p), ("scale", C.c_void_p), ("group_size", C.c_size_t)]


class RbtActivation(C.Structure):
    _fields_ = [("kind", C.c_int32), ("beta", C.c_float), ("linear_beta", C.c_float),
                ("has_linear_beta", C.c_int32)]


class RbtExpertSlot(C.Structure):
    _fields_ = [("eid", C.c_uint32), ("fused", C.c_int32), ("gate", RbtQT), ("up", RbtQT),
                ("gate_up", RbtQT), ("down", RbtQT)]


class RbtLatentMoeDesc(C.Structure):
    _fields_ = [("moe_hidden", C.c_size_t), ("down_proj", RbtQT), ("up_proj", RbtQT), ("norm", C.c_void_p),
                ("eps", C.c_float), ("act", RbtActivation)]


class RbtMoeLayerDesc(C.Structure):
    _fields_ = [("family", C.c_int32), ("hidden", C.c_size_t), ("moe_inter", C.c_size_t),
                ("n_experts", C.c_size_t), ("topk", C.c_size_t), ("router", C.c_void_p),
                ("router_bias", C.c_void_p), ("logit_bias", C.c_void_p), ("norm_topk", C.c_int32),
                ("routed_scale", C.c_float), ("n_group", C.c_size_t), ("topk_group", C.c_size_t),
                ("has_shared", C.c_int32), ("shared", RbtExpertSlot), ("shared_gate", C.c_void_p)]


class RbtProfile(C.Structure):
    _fields_ = [("router_ms", C.c_double), ("gateup_ms", C.c_double), ("down_ms", C.c_double),
                ("combine_ms", C.c_double), ("calls", C.c_uint64), ("ambiguous", C.c_uint64),
                ("gateup_experts", C.c_uint64), ("down_experts", C.c_uint64)]


_P, _S, _I, _F, _U32, _U64 = C.c_void_p, C.c_size_t, C.c_int32, C.c_float, C.c_uint32, C.c_uint64
_CTX = C.c_void_p


class RbtGdnDesc(C.Structure):
    _fields_ = [("n_v_heads", C.c_size_t), ("n_k_heads", C.c_size_t), ("head_k_dim", C.c_size_t),
                ("head_v_dim", C.c_size_t), ("conv_kernel", C.c_size_t), ("conv_weight", C.c_void_p),
                ("a_log", C.c_void_p), ("dt_bias", C.c_void_p), ("norm_weight", C.c_void_p), ("eps", C.c_float)]


class RbtGqaDesc(C.Structure):
    _fields_ = [("n_heads", C.c_size_t), ("n_kv_heads", C.c_size_t), ("head_dim", C.c_size_t),
                ("rope_dim", C.c_size_t), ("theta", C.c_float), ("attn_scale", C.c_float), ("eps", C.c_float),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


class RbtKernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 160), ("launches", C.c_uint64), ("total_ms", C.c_double)]


class RbtTensorInfo(C.Structure):
    _fields_ = [("file_index", C.c_int32), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("dtype", C.c_char * 16), ("ndim", C.c_int32), ("shape", C.c_uint64 * 8)]


NAMING_QWEN38_MXFP4, NAMING_KIMI_K3_MXFP4 = 0, 1

# name -> (restype, argtypes)
SIGNATURES = {
    "rbt_init": (_I, [C.POINTER(C.c_void_p), C.c_int]),
    "rbt_destroy": (None, [_CTX]),
    "rbt_last_error": (C.c_char_p, [_CTX]),
    "rbt_sync": (_I, [_CTX]),
    "rbt_stream": (C.c_void_p, [_CTX]),
    "rbt_version": (C.c_char_p, []),
    "rbt_qt_resident_bytes": (_S, [C.POINTER(RbtQT)]),
    "rbt_dequant_rows": (_I, [_CTX, C.POINTER(RbtQT), _S, _S, _P]),
    "rbt_dequant_rows_d": (_I, [_CTX, C.POINTER(RbtQT), _S, _S, _P]),
    "rbt_matmul": (_I, [_CTX, _P, _P, _P, _S, _S, _S]),
    "rbt_matmul_d": (_I, [_CTX, _P, _P, _P, _S, _S, _S]),
    "rbt_matmul_mxfp4": (_I, [_CTX, _P, _P, _P, _P, _S, _S, _S]),
    "rbt_matmul_mxfp4_d": (_I, [_CTX, _P, _P, _P, _P, _S, _S, _S]),
    "rbt_matmul_i4_grouped": (_I, [_CTX, _P, _P, _P, _P, _S, _S, _S, _S]),
    "rbt_matmul_i4_grouped_d": (_I, [_CTX, _P, _P, _P, _P, _S, _S, _S, _S]),
    "rbt_matmul_qt": (_I, [_CTX, _P, _P, C.POINTER(RbtQT), _S]),
    "rbt_matmul_qt_d": (_I, [_CTX, _P, _P, C.POINTER(RbtQT), _S]),
    "rbt_route_softmax_topk": (_I, [_CTX, _P, _S, _S, _S, _P, _P]),
    "rbt_route_softmax_topk_d": (_I, [_CTX, _P, _S, _S, _S, _P, _P]),
    "rbt_route_sigmoid_topk": (_I, [_CTX, _P, _P, _S, _S, _S, _I, _F, _S, _S, _P, _P]),
    "rbt_route_sigmoid_topk_d": (_I, [_CTX, _P, _P, _S, _S, _S, _I, _F, _S, _S, _P, _P]),
    "rbt_unique_experts": (_I, [_P, _S, _S, _P]),
    "rbt_apply_single_expert": (_I, [_CTX, C.POINTER(RbtExpertSlot), _P, _P, _S, _S, _P, _S, _S, _I, _P]),
    "rbt_apply_single_expert_d": (_I, [_CTX, C.POINTER(RbtExpertSlot), _P, _P, _S, _S, _P, _S, _S, _I, _P]),
    "rbt_apply_single_expert_act": (_I, [_CTX, C.POINTER(RbtExpertSlot), _P, _P, _S, _S, _P, _S, _S,
                                         C.POINTER(RbtActivation), _P]),
    "rbt_apply_single_expert_act_d": (_I, [_CTX, C.POINTER(RbtExpertSlot), _P, _P, _S, _S, _P, _S, _S,
                                           C.POINTER(RbtActivation), _P]),
    "rbt_latent_moe_d": (_I, [_CTX, _U32, C.POINTER(RbtLatentMoeDesc), _P, _S, _P, _P, _P]),
    "rbt_pool_put": (_I, [_CTX, _U32, C.POINTER(RbtExpertSlot)]),
    "rbt_pool_put_device": (_I, [_CTX, _U32, C.POINTER(RbtExpertSlot)]),
    "rbt_pool_alloc": (C.POINTER(RbtExpertSlot), [_CTX, _U32, _U32, _I, _S, _S, _S]),
    "rbt_pool_get": (C.POINTER(RbtExpertSlot), [_CTX, _U32, _U32]),
    "rbt_pool_resident_bytes": (_S, [_CTX]),
    "rbt_moe_layer_set": (_I, [_CTX, _U32, C.POINTER(RbtMoeLayerDesc)]),
    "rbt_moe_layer_set_device": (_I, [_CTX, _U32, C.POINTER(RbtMoeLayerDesc)]),
    "rbt_moe_forward": (_I, [_CTX, _U32, _P, _S, _P, _P, _P]),
    "rbt_moe_forward_d": (_I, [_CTX, _U32, _P, _S, _P, _P, _P]),
    "rbt_moe_forward_noalloc_d": (_I, [_CTX, _U32, _P, _S, _P, _P, _P]),
    "rbt_shards_open": (_I, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "rbt_shards_close": (None, [C.c_void_p]),
    "rbt_shards_last_error": (C.c_char_p, []),
    "rbt_shards_count": (_S, [C.c_void_p]),
    "rbt_shards_find": (_I, [C.c_void_p, C.c_char_p, C.POINTER(RbtTensorInfo)]),
    "rbt_shards_read": (_I, [C.c_void_p, C.c_char_p, _P, _S]),
    "rbt_shards_read_range": (_I, [C.c_void_p, C.c_char_p, _U64, _P, _S]),
    "rbt_pool_load_mxfp4": (_I, [_CTX, C.c_void_p, _I, _U32, _P, _S, _S, _S]),
    "rbt_rmsnorm_d": (_I, [_CTX, _P, _P, _S, _S, _F]),
    "rbt_rmsnorm_1p_d": (_I, [_CTX, _P, _P, _S, _S, _F]),
    "rbt_moe_sublayer": (_I, [_CTX, _U32, _P, _S, _P, _F, _P, _P]),
    "rbt_moe_sublayer_d": (_I, [_CTX, _U32, _P, _S, _P, _F, _P, _P]),
    "rbt_gdn_step_d": (_I, [_CTX, C.POINTER(RbtGdnDesc), _P, _P, _P, _P, _P, _P, _P]),
    "rbt_gqa_step_d": (_I, [_CTX, C.POINTER(RbtGqaDesc), _P, _P, _S, _S, _P, _P, _P, _P]),
    "rbt_profile_enable": (_I, [_CTX, _I]),
    "rbt_profile_read": (_I, [_CTX, C.POINTER(RbtProfile), _I]),
    "rbt_profile_kernels": (_I, [_CTX, _I]),
    "rbt_profile_kernels_read": (_I, [_CTX, C.POINTER(RbtKernelStat), _S, C.POINTER(C.c_size_t), _I]),
    "rbt_synth_mxfp4_d": (_I, [_CTX, _P, _P, _S, _S, _U64, _U32, _U32]),
    "rbt_synth_i4g_d": (_I, [_CTX, _P, _P, _S, _S, _S, _U64, _F, _F]),
}

_lib = None


def header_symbols(path: str = HEADER) -> list[str]:
    """Every function name declared in include/rabbit_amd.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rbt_[a-z0-9_]+)\s*\(", text)))


def load(path: str = LIB_PATH):
    """Loads librabbit_amd.so and declares every signature. Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                           "or `python rabbit_amd/build.py` (there is no CPU fallback)")
    # One HIP runtime per process: PyTorch-ROCm ships its own libamdhip64 (SONAME libamdhip64.so.7).
    # Importing torch first makes this library bind to that already-loaded runtime; loading ours
    # first would pull /opt/rocm's copy in beside torch's, and the second runtime finds no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError = the build lacks a declared symbol
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
