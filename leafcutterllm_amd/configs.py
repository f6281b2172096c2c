"""The benchmark layer shapes and their seeded synthetic weights.

Five shapes: a small Q8_0 layer, a Mixtral-8x7B-shaped Q4_K layer, a
fine-grained Qwen-MoE-shaped prefill layer with shared experts and a skewing
router bias, a DeepSeek-V3-shaped sigmoid/group-routed layer with a Q6_K down
projection, and the per-layer shape of the end-to-end synthetic model.

Synthetic data contract (the bytes are the contract, not the floats):
  element i of stream (seed, kind << 32 | index) = counter-based splitmix64 +
  Box-Muller (lcmoe_synth_normal); activations N(0,1), weights N(0, 0.02)
  quantised with lcmoe_quantize, router f32 N(0, 0.02), DeepSeek bias
  N(0, 0.1), prefill-layer bias +2.0 on experts 0..7.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from ._lib import (ROUTE_SIGMOID_GROUP, ROUTE_SOFTMAX, ROUTE_SOFTMAX_RENORM, TYPE_Q4_K,
                   TYPE_Q6_K, TYPE_Q8_0, Desc, check, lib)

# stream kinds
S_X, S_ROUTER, S_BIAS, S_GATE, S_UP, S_DOWN, S_GATE_SH, S_UP_SH, S_DOWN_SH = range(9)
WEIGHT_STD = 0.02


def stream(kind: int, index: int = 0) -> int:
    return (kind << 32) | index


@dataclass
class LayerConfig:
    name: str
    d_model: int
    d_ff: int
    n_expert: int
    n_expert_used: int
    route_kind: int
    qtype_gate: int
    qtype_down: int
    n_shared: int = 0
    d_ff_shared: int = 0
    n_group: int = 0
    topk_group: int = 0
    routed_scale: float = 1.0
    bias: str = "none"  # none | plus2_first8 | normal0.1
    tokens: tuple = (1,)
    note: str = ""
    extra: dict = field(default_factory=dict)

    def desc(self, max_tokens: int) -> Desc:
        d = Desc()
        d.d_model, d.d_ff = self.d_model, self.d_ff
        d.n_expert, d.n_expert_used = self.n_expert, self.n_expert_used
        d.n_shared, d.d_ff_shared = self.n_shared, self.d_ff_shared
        d.route_kind, d.n_group, d.topk_group = self.route_kind, self.n_group, self.topk_group
        d.routed_scale = self.routed_scale
        d.has_bias = 0 if self.bias == "none" else 1
        d.type_gate = d.type_up = self.qtype_gate
        d.type_down = self.qtype_down
        d.type_gate_sh = d.type_up_sh = self.qtype_gate if self.n_shared else 0
        d.type_down_sh = self.qtype_down if self.n_shared else 0
        d.max_tokens = max_tokens
        return d

    def expert_bytes(self) -> int:
        ts = tensor_size
        return (2 * ts(self.qtype_gate, self.d_ff * self.d_model)
                + ts(self.qtype_down, self.d_model * self.d_ff))

    def shared_bytes(self) -> int:
        ts = tensor_size
        return (2 * ts(self.qtype_gate, self.d_ff_shared * self.d_model)
                + ts(self.qtype_down, self.d_model * self.d_ff_shared))

    def layer_bytes(self) -> int:
        return (self.n_expert * self.expert_bytes() + self.n_shared * self.shared_bytes()
                + 4 * self.d_model * self.n_expert)


CONFIGS = {
    1: LayerConfig("q8_0-d1024-e8k2", 1024, 2816, 8, 2, ROUTE_SOFTMAX_RENORM, TYPE_Q8_0, TYPE_Q8_0,
                   tokens=(1, 16), note="Single MoE FFN layer, Q8_0 experts"),
    2: LayerConfig("mixtral-8x7b-q4_k", 4096, 14336, 8, 2, ROUTE_SOFTMAX_RENORM, TYPE_Q4_K,
                   TYPE_Q4_K, tokens=(1, 8, 64), note="Mixtral-8x7B-shaped MoE layer, Q4_K"),
    3: LayerConfig("qwen-moe-prefill-q4_k", 2048, 1408, 60, 4, ROUTE_SOFTMAX, TYPE_Q4_K, TYPE_Q4_K,
                   n_shared=4, d_ff_shared=1408, bias="plus2_first8", tokens=(2048,),
                   note="Fine-grained prefill layer, +2.0 bias on experts 0..7"),
    4: LayerConfig("deepseek-v3-q4_k-q6_k", 7168, 2048, 256, 8, ROUTE_SIGMOID_GROUP, TYPE_Q4_K,
                   TYPE_Q6_K, n_shared=1, d_ff_shared=2048, n_group=8, topk_group=4,
                   routed_scale=2.5, bias="normal0.1", tokens=(1, 32, 256),
                   note="DeepSeek-V3-shaped layer, sigmoid group-limited routing"),
    5: LayerConfig("e2e-layer-q4_k", 2048, 1408, 60, 4, ROUTE_SOFTMAX, TYPE_Q4_K, TYPE_Q4_K,
                   n_shared=4, d_ff_shared=1408, tokens=(1, 16),
                   note="per-layer MoE shape of the 24-layer end-to-end decode model"),
}


def tensor_size(qtype: int, count: int) -> int:
    return int(lib().lcmoe_tensor_size(qtype, count))


def synth_normal(seed: int, strm: int, std: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().lcmoe_synth_normal(seed, strm, std, out.ctypes.data, n)
    return out


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(tensor_size(qtype, x.size), np.uint8)
    check(lib().lcmoe_quantize(qtype, x.ctypes.data, out.ctypes.data, x.size), "lcmoe_quantize")
    return out


def _stacked(qtype: int, rows: int, cols: int, n: int, seed: int, kind: int) -> np.ndarray:
    sz = tensor_size(qtype, rows * cols)
    out = np.empty(n * sz, np.uint8)
    for e in range(n):
        w = synth_normal(seed, stream(kind, e), WEIGHT_STD, rows * cols)
        check(lib().lcmoe_quantize(qtype, w.ctypes.data, out[e * sz:].ctypes.data, w.size),
              "lcmoe_quantize")
    return out


def synth_layer(cfg: LayerConfig, seed: int = 0) -> dict:
    """Seeded synthetic layer: numpy arrays keyed like lcmoe_weights."""
    d, F, E = cfg.d_model, cfg.d_ff, cfg.n_expert
    layer = {
        "router": synth_normal(seed, stream(S_ROUTER), WEIGHT_STD, d * E).reshape(d, E),
        "bias": None,
        "gate": _stacked(cfg.qtype_gate, F, d, E, seed, S_GATE),
        "up": _stacked(cfg.qtype_gate, F, d, E, seed, S_UP),
        "down": _stacked(cfg.qtype_down, d, F, E, seed, S_DOWN),
    }
    if cfg.bias == "plus2_first8":
        b = np.zeros(E, np.float32)
        b[:8] = 2.0
        layer["bias"] = b
    elif cfg.bias == "normal0.1":
        layer["bias"] = synth_normal(seed, stream(S_BIAS), 0.1, E)
    if cfg.n_shared:
        FS, S = cfg.d_ff_shared, cfg.n_shared
        layer["gate_sh"] = _stacked(cfg.qtype_gate, FS, d, S, seed, S_GATE_SH)
        layer["up_sh"] = _stacked(cfg.qtype_gate, FS, d, S, seed, S_UP_SH)
        layer["down_sh"] = _stacked(cfg.qtype_down, d, FS, S, seed, S_DOWN_SH)
    return layer


def synth_x(cfg: LayerConfig, T: int, seed: int = 0, index: int = 0) -> np.ndarray:
    return synth_normal(seed, stream(S_X, index), 1.0, T * cfg.d_model).reshape(T, cfg.d_model)


def small_config(name: str, d: int, F: int, E: int, K: int, route_kind: int, qg: int, qd: int,
                 **kw) -> LayerConfig:
    """A reduced shape with the same semantics, for fast parity tests."""
    return LayerConfig(name, d, F, E, K, route_kind, qg, qd, **kw)


# ---- end-to-end decoder model -----------------------------------------------

S_EMBD, S_OUT, S_NORM, S_ATTN = 16, 17, 18, 19  # stream kinds of the model tensors


@dataclass
class ModelConfig:
    """A decoder model around the MoE layer `layer` (the engine of
    rust/src/inference/engine.rs:78-132 with an MoE FFN)."""
    name: str
    n_layer: int
    n_head: int
    n_kv_head: int
    head_dim: int
    vocab: int
    rope_theta: float
    layer: LayerConfig
    attn_type: int = TYPE_Q4_K
    note: str = ""

    @property
    def d_model(self) -> int:
        return self.layer.d_model

    def desc(self, max_batch: int, max_prompt: int, max_ctx: int, rope_positions: int = 0,
             n_layer: int = 0):
        from .model import ModelDesc
        d = ModelDesc()
        d.n_layer = n_layer or self.n_layer
        d.d_model, d.n_head, d.n_kv_head = self.d_model, self.n_head, self.n_kv_head
        d.head_dim, d.vocab, d.rope_theta, d.norm_eps = self.head_dim, self.vocab, self.rope_theta, 1e-5
        d.rope_positions, d.attn_type = rope_positions, self.attn_type
        d.max_batch, d.max_prompt, d.max_ctx = max_batch, max_prompt, max_ctx
        d.moe = self.layer.desc(max(max_batch, max_prompt))
        return d

    def layer_bytes(self) -> int:
        """Resident bytes of one decoder layer's weights."""
        d, qd, kvd = self.d_model, self.n_head * self.head_dim, self.n_kv_head * self.head_dim
        ts = tensor_size
        attn = ts(self.attn_type, (qd + 2 * kvd) * d) + ts(self.attn_type, d * qd)
        return attn + self.layer.layer_bytes() + 8 * d


MODEL_CONFIGS = {
    # 24 layers, d_model 2048, 16 heads x 128 with RoPE,
    # the config-5 MoE layer (60 experts top-4 + 4 shared, d_ff 1408), vocab
    # 32000, every matrix Q4_K.  RoPE base: the reference's default
    # (ModelConfig::default, rust/src/model/loader.rs:24-36).
    5: ModelConfig("e2e-moe-24l-q4_k", 24, 16, 16, 128, 32000, 10000.0, CONFIGS[5],
                   note="24-layer synthetic MoE decoder, Q4_K"),
}


def synth_model(mc: ModelConfig, seed: int = 0, n_layer: int = 0) -> dict:
    """Seeded synthetic model weights (N(0, 0.02) matrices quantised to
    mc.attn_type / the MoE types, norm weights 1 + N(0, 0.02)), keyed as
    Model and the oracle's engine take them; layer l's MoE is
    synth_layer(mc.layer, seed * 1000 + l)."""
    n_layer = n_layer or mc.n_layer
    d, V = mc.d_model, mc.vocab
    qd, kvd = mc.n_head * mc.head_dim, mc.n_kv_head * mc.head_dim

    def mat(rows, cols, kind, index):
        return quantize(mc.attn_type, synth_normal(seed, stream(kind, index), WEIGHT_STD, rows * cols))

    def norm(index):
        return 1.0 + synth_normal(seed, stream(S_NORM, index), WEIGHT_STD, d)

    layers = []
    for l in range(n_layer):
        layers.append({
            "attn_norm": norm(2 * l), "ffn_norm": norm(2 * l + 1),
            "attn_q": mat(qd, d, S_ATTN, 4 * l), "attn_k": mat(kvd, d, S_ATTN, 4 * l + 1),
            "attn_v": mat(kvd, d, S_ATTN, 4 * l + 2), "attn_o": mat(d, qd, S_ATTN, 4 * l + 3),
            "moe": synth_layer(mc.layer, seed=seed * 1000 + l),
        })
    return {"token_embd": mat(V, d, S_EMBD, 0), "output": mat(V, d, S_OUT, 0),
            "output_norm": norm(1 << 20), "layers": layers}


__all__ = ["CONFIGS", "LayerConfig", "synth_layer", "synth_x", "synth_normal", "quantize",
           "tensor_size", "stream", "small_config", "C", "ModelConfig", "MODEL_CONFIGS",
           "synth_model"]
