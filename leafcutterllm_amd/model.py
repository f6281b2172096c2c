"""Host-side mirror of the reference engine over the C ABI (lcmoe_model_*).

`Model` has the surface of the reference's Engine
(rust/src/inference/engine.rs:10-132): `forward(tokens)` returns the last
token's logits and appends to the KV cache, `generate(prompt, n)` is the
greedy generate loop, `reset()` is KVCache::clear.  It extends them to a
batch of sequences decoded together.  All compute runs in liblcmoe.so on the
GPU; this module only packs pointers.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import Desc, LcmoeError, Weights, check, lib

ROPE_PER_CALL, ROPE_ABSOLUTE = 0, 1


class ModelDesc(C.Structure):
    """lcmoe_model_desc (include/lcmoe.h)."""

    _fields_ = [
        ("n_layer", C.c_int32), ("d_model", C.c_int32), ("n_head", C.c_int32),
        ("n_kv_head", C.c_int32), ("head_dim", C.c_int32), ("vocab", C.c_int32),
        ("rope_theta", C.c_float), ("norm_eps", C.c_float), ("rope_positions", C.c_int32),
        ("attn_type", C.c_int32), ("max_batch", C.c_int32), ("max_prompt", C.c_int32),
        ("max_ctx", C.c_int32), ("moe", Desc),
    ]


class LayerWeights(C.Structure):
    """lcmoe_layer_weights."""

    _fields_ = [
        ("attn_norm", C.c_void_p), ("attn_q", C.c_void_p), ("attn_k", C.c_void_p),
        ("attn_v", C.c_void_p), ("attn_o", C.c_void_p), ("ffn_norm", C.c_void_p),
        ("moe", Weights),
    ]


class ModelWeights(C.Structure):
    """lcmoe_model_weights."""

    _fields_ = [
        ("token_embd", C.c_void_p), ("output_norm", C.c_void_p), ("output", C.c_void_p),
        ("layers", C.c_void_p),
    ]


_SIGS = {
    "lcmoe_model_create": (C.c_int32, [C.POINTER(ModelDesc), C.POINTER(ModelWeights),
                                       C.POINTER(C.c_void_p)]),
    "lcmoe_model_destroy": (None, [C.c_void_p]),
    "lcmoe_model_reset": (C.c_int32, [C.c_void_p]),
    "lcmoe_model_forward": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                        C.c_void_p]),
    "lcmoe_model_generate": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                         C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]),
    "lcmoe_model_last_timing": (C.c_int32, [C.c_void_p, C.POINTER(C.c_double),
                                            C.POINTER(C.c_double)]),
    "lcmoe_model_set_decode_graph": (C.c_int32, [C.c_void_p, C.c_int32]),
    "lcmoe_model_debug_fail_forward": (C.c_int32, [C.c_void_p, C.c_int32]),
    "lcmoe_model_debug_layer_moe": (C.c_int32, [C.c_void_p, C.c_int32, C.POINTER(C.c_void_p)]),
}


def _bound():
    L = lib()
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data


class Model:
    """A resident decoder model on the current HIP device.

    `weights` holds numpy arrays: token_embd / output (GGUF bytes [vocab,
    d]; output absent or None ties the LM head to token_embd), output_norm (f32 [d]) and `layers`, a list of dicts with attn_norm,
    ffn_norm (f32 [d]), attn_q / attn_k / attn_v / attn_o (GGUF bytes) and
    `moe` (the arrays lcmoe_create takes: router, bias, gate, up, down and
    the *_sh tensors)."""

    def __init__(self, desc: ModelDesc, weights: dict):
        L = _bound()
        self.desc = desc
        keep = []

        def p(a, dt):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dt)
            keep.append(a)
            return a.ctypes.data

        layers = (LayerWeights * desc.n_layer)()
        for i, lw in enumerate(weights["layers"]):
            lay = layers[i]
            lay.attn_norm, lay.ffn_norm = p(lw["attn_norm"], np.float32), p(lw["ffn_norm"], np.float32)
            for k in ("attn_q", "attn_k", "attn_v", "attn_o"):
                setattr(lay, k, p(lw[k], np.uint8))
            m = lw["moe"]
            lay.moe.router, lay.moe.bias = p(m["router"], np.float32), p(m.get("bias"), np.float32)
            for k in ("gate", "up", "down", "gate_sh", "up_sh", "down_sh"):
                setattr(lay.moe, k, p(m.get(k), np.uint8))
        w = ModelWeights()
        w.token_embd = p(weights["token_embd"], np.uint8)
        w.output = p(weights.get("output"), np.uint8)  # None: tied to token_embd
        w.output_norm = p(weights["output_norm"], np.float32)
        w.layers = C.cast(layers, C.c_void_p)
        h = C.c_void_p()
        check(L.lcmoe_model_create(C.byref(desc), C.byref(w), C.byref(h)), "lcmoe_model_create")
        self._h = h

    def reset(self) -> None:
        check(_bound().lcmoe_model_reset(self._h), "lcmoe_model_reset")

    def forward(self, tokens) -> np.ndarray:
        """Engine::forward for each row of tokens [B, T]: logits [B, vocab]."""
        t = np.ascontiguousarray(np.atleast_2d(tokens), np.int32)
        B, T = t.shape
        out = np.empty((B, self.desc.vocab), np.float32)
        check(_bound().lcmoe_model_forward(self._h, t.ctypes.data, B, T, out.ctypes.data),
              "lcmoe_model_forward")
        return out

    def generate(self, prompt, n_new: int, eos: int = -1):
        """Greedy Engine::generate for each row of prompt [B, P]: (ids [B,
        n_new], count per row up to and including the first eos)."""
        pr = np.ascontiguousarray(np.atleast_2d(prompt), np.int32)
        B, P = pr.shape
        out = np.empty((B, n_new), np.int32)
        n = np.empty(B, np.int32)
        check(_bound().lcmoe_model_generate(self._h, pr.ctypes.data, B, P, n_new, eos,
                                            out.ctypes.data, n.ctypes.data),
              "lcmoe_model_generate")
        return out, n

    def set_decode_graph(self, enable: bool) -> None:
        check(_bound().lcmoe_model_set_decode_graph(self._h, int(enable)),
              "lcmoe_model_set_decode_graph")

    def debug_fail_forward(self, n: int) -> None:
        """Testing of the error path: the n-th internal forward from now on
        fails before enqueueing anything (lcmoe_model_debug_fail_forward)."""
        check(_bound().lcmoe_model_debug_fail_forward(self._h, int(n)),
              "lcmoe_model_debug_fail_forward")

    def layer_routing(self, layer: int) -> dict:
        """Routing of layer `layer`'s most recent MoE forward (observation:
        lcmoe_model_debug_layer_moe + lcmoe_get_dispatch): topk_idx, topk_w
        [T, K]."""
        h = C.c_void_p()
        check(_bound().lcmoe_model_debug_layer_moe(self._h, int(layer), C.byref(h)),
              "lcmoe_model_debug_layer_moe")
        K, cap = self.desc.moe.n_expert_used, max(self.desc.max_batch, self.desc.max_prompt)
        T = C.c_int32()
        idx = np.empty((cap, K), np.int32)
        w = np.empty((cap, K), np.float32)
        check(lib().lcmoe_get_dispatch(h, C.byref(T), idx.ctypes.data, w.ctypes.data, None, None,
                                       None, None), "lcmoe_get_dispatch")
        return {"topk_idx": idx[:T.value].copy(), "topk_w": w[:T.value].copy()}

    def last_timing(self):
        a, b = C.c_double(), C.c_double()
        check(_bound().lcmoe_model_last_timing(self._h, C.byref(a), C.byref(b)),
              "lcmoe_model_last_timing")
        return a.value, b.value

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _bound().lcmoe_model_destroy(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["Model", "ModelDesc", "LayerWeights", "ModelWeights", "ROPE_PER_CALL", "ROPE_ABSOLUTE",
           "LcmoeError"]
