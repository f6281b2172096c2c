"""ctypes binding of the product library leafcutterllm_amd/liblcmoe.so.

The library must have been built (leafcutterllm_amd/build.py, or
__graft_entry__.build()).  A missing library is an error: there is no
fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# LCMOE_LIB names another build of the same library (e.g. a variant being
# timed); the default is the in-tree build
LIB_PATH = os.environ.get("LCMOE_LIB") or os.path.join(_HERE, "liblcmoe.so")

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 8, 12, 14
TYPE_Q4_0 = 2  # lcmoe_shard_matmul only: the shard engine's interleaved Q4_0
ROUTE_SOFTMAX_RENORM, ROUTE_SOFTMAX, ROUTE_SIGMOID_GROUP = 0, 1, 2
ACT_F16, ACT_F16X2 = 0, 1  # lcmoe_set_act_precision

STATUS = {
    0: "LCMOE_OK", 1: "LCMOE_ERR_INVALID_ARG", 2: "LCMOE_ERR_UNSUPPORTED",
    3: "LCMOE_ERR_CORRUPT", 4: "LCMOE_ERR_HIP", 5: "LCMOE_ERR_OUT_OF_MEMORY",
    6: "LCMOE_ERR_STATE", 7: "LCMOE_ERR_NOT_FOUND", 8: "LCMOE_ERR_IO",
}

# every symbol include/lcmoe.h declares
EXPORTS = (
    "lcmoe_create", "lcmoe_destroy", "lcmoe_forward", "lcmoe_forward_dev",
    "lcmoe_get_dispatch", "lcmoe_set_timing", "lcmoe_get_timing", "lcmoe_timing_name",
    "lcmoe_timing_slots", "lcmoe_last_error", "lcmoe_tensor_size", "lcmoe_scan_blocks",
    "lcmoe_quantize", "lcmoe_synth_normal", "lcmoe_debug_dequant", "lcmoe_debug_sigmoid",
    "lcmoe_gguf_open", "lcmoe_gguf_close", "lcmoe_gguf_meta_int", "lcmoe_gguf_meta_str",
    "lcmoe_gguf_tensor", "lcmoe_gguf_block_count", "lcmoe_gguf_is_moe_layer",
    "lcmoe_gguf_moe_layer", "lcmoe_set_norm", "lcmoe_forward_norm_residual",
    "lcmoe_forward_norm_residual_dev", "lcmoe_debug_rmsnorm", "lcmoe_shard_matmul",
    "lcmoe_shard_matmul_dev", "lcmoe_shard_matmul_split_dev",
    "lcmoe_shard_matmul_split_noalloc_dev", "lcmoe_model_create", "lcmoe_model_destroy",
    "lcmoe_model_reset", "lcmoe_model_forward", "lcmoe_model_generate",
    "lcmoe_model_last_timing", "lcmoe_model_set_decode_graph", "lcmoe_matmul_f32",
    "lcmoe_matmul_f32_dev", "lcmoe_debug_route_fallbacks", "lcmoe_debug_read_bandwidth",
    "lcmoe_dequantize", "lcmoe_sanitize_blocks", "lcmoe_model_debug_fail_forward",
    "lcmoe_model_debug_layer_moe", "lcmoe_set_act_precision",
)


class Desc(C.Structure):
    """lcmoe_desc (include/lcmoe.h)."""

    _fields_ = [
        ("d_model", C.c_int32), ("d_ff", C.c_int32), ("n_expert", C.c_int32),
        ("n_expert_used", C.c_int32), ("n_shared", C.c_int32), ("d_ff_shared", C.c_int32),
        ("route_kind", C.c_int32), ("n_group", C.c_int32), ("topk_group", C.c_int32),
        ("routed_scale", C.c_float), ("has_bias", C.c_int32),
        ("type_gate", C.c_int32), ("type_up", C.c_int32), ("type_down", C.c_int32),
        ("type_gate_sh", C.c_int32), ("type_up_sh", C.c_int32), ("type_down_sh", C.c_int32),
        ("max_tokens", C.c_int32),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class Weights(C.Structure):
    """lcmoe_weights (include/lcmoe.h)."""

    _fields_ = [
        ("router", C.c_void_p), ("bias", C.c_void_p),
        ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
        ("gate_sh", C.c_void_p), ("up_sh", C.c_void_p), ("down_sh", C.c_void_p),
    ]


class LcmoeError(RuntimeError):
    def __init__(self, status: int, where: str, message: str):
        self.status = status
        super().__init__(f"{where}: {STATUS.get(status, status)}: {message}")


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run leafcutterllm_amd/build.py "
                           "(or __graft_entry__.build()) first")
    L = C.CDLL(LIB_PATH)
    vp, i32, i64, u64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float
    P = C.POINTER
    sigs = {
        "lcmoe_create": (i32, [P(Desc), P(Weights), P(vp)]),
        "lcmoe_destroy": (None, [vp]),
        "lcmoe_forward": (i32, [vp, vp, i32, vp, vp, vp]),
        "lcmoe_forward_dev": (i32, [vp, vp, i32, vp, vp]),
        "lcmoe_get_dispatch": (i32, [vp, vp, vp, vp, vp, vp, vp, vp]),
        "lcmoe_set_timing": (i32, [vp, i32]),
        "lcmoe_get_timing": (i32, [vp, i32, vp, vp]),
        "lcmoe_timing_name": (C.c_char_p, [i32]),
        "lcmoe_timing_slots": (i32, []),
        "lcmoe_last_error": (C.c_char_p, []),
        "lcmoe_tensor_size": (C.c_size_t, [i32, i64]),
        "lcmoe_scan_blocks": (i64, [i32, vp, i64]),
        "lcmoe_dequantize": (i64, [i32, vp, i64, vp, i32]),
        "lcmoe_sanitize_blocks": (i64, [i32, vp, i64, P(i64)]),
        "lcmoe_quantize": (i32, [i32, vp, vp, i64]),
        "lcmoe_synth_normal": (None, [u64, u64, f32, vp, i64]),
        "lcmoe_debug_dequant": (i32, [i32, vp, i64, vp]),
        "lcmoe_debug_sigmoid": (i32, [vp, i64, vp]),
        "lcmoe_debug_route_fallbacks": (i32, [vp, vp]),
        "lcmoe_debug_read_bandwidth": (i32, [i64, i32, vp]),
        "lcmoe_debug_rmsnorm": (i32, [vp, vp, f32, i32, i32, vp]),
        "lcmoe_set_norm": (i32, [vp, vp, f32]),
        "lcmoe_set_act_precision": (i32, [vp, i32]),
        "lcmoe_shard_matmul": (i32, [i32, vp, vp, vp, i32, i32, i32]),
        "lcmoe_shard_matmul_dev": (i32, [i32, vp, vp, vp, i32, i32, i32, vp]),
        "lcmoe_shard_matmul_split_dev": (i32, [i32, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
        "lcmoe_shard_matmul_split_noalloc_dev": (i32, [i32, vp, vp, vp, i32, i32, i32, i32, vp]),
        "lcmoe_matmul_f32": (i32, [vp, vp, vp, i32, i32, i32]),
        "lcmoe_matmul_f32_dev": (i32, [vp, vp, vp, i32, i32, i32, vp]),
        "lcmoe_forward_norm_residual": (i32, [vp, vp, i32, vp, vp, vp]),
        "lcmoe_forward_norm_residual_dev": (i32, [vp, vp, i32, vp, vp]),
        "lcmoe_gguf_open": (i32, [C.c_char_p, P(vp)]),
        "lcmoe_gguf_close": (None, [vp]),
        "lcmoe_gguf_meta_int": (i32, [vp, C.c_char_p, P(i64)]),
        "lcmoe_gguf_meta_str": (C.c_char_p, [vp, C.c_char_p]),
        "lcmoe_gguf_tensor": (i32, [vp, C.c_char_p, P(i32), P(i32), P(i64), P(vp), P(u64)]),
        "lcmoe_gguf_block_count": (i32, [vp]),
        "lcmoe_gguf_is_moe_layer": (i32, [vp, i32]),
        "lcmoe_gguf_moe_layer": (i32, [vp, i32, i32, P(Desc), P(Weights)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(status: int, where: str) -> None:
    if status != 0:
        msg = lib().lcmoe_last_error()
        raise LcmoeError(status, where, msg.decode() if msg else "")
