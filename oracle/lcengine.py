"""CPU restatement of the reference engine's decoder forward and greedy
generation, composed from the oracle's restated kernels.

TEST INFRASTRUCTURE ONLY: the checker of the end-to-end engine
(lcmoe_model_*); imported by tests/ and nothing in the product.

It follows rust/src/inference/engine.rs:51-132 statement by statement, with
the MoE FFN (lco_moe_forward) in place of the dense ffn_forward at
engine.rs:114:
  embed_lookup (engine.rs:134-144: rows of the dequantised table, zeros for
  an id past the vocabulary), then per layer rms_norm (cpu.rs:49-60) ->
  attention_forward (attention.rs:37-118: q/k/v = x W, RoPE, f16 KV cache
  append, masked softmax attention, o = a W_o) -> residual add ->
  rms_norm -> MoE FFN -> residual add; the final rms_norm; the lm_head
  product of the last token; greedy sample_top_p (sampler.rs:8-10).
Weights enter as GGUF bytes and are ingested as load_layer does
(loader.rs:145-168: dequantise, transpose 2D to [in, out], sanitize); the
embedding is not transposed (loader.rs:185-187).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import lcoracle as O

ROPE_PER_CALL, ROPE_ABSOLUTE = 0, 1


@dataclass
class ModelSpec:
    n_layer: int
    d_model: int
    n_head: int
    n_kv_head: int
    head_dim: int
    vocab: int
    rope_theta: float
    attn_type: int           # GGUF type of the q/k/v/o, embedding and output tensors
    moe_desc: O.Desc
    eps: float = 1e-5
    rope_positions: int = ROPE_PER_CALL
    extra: dict = field(default_factory=dict)


def ingest(qtype: int, data: np.ndarray, rows: int, cols: int, transpose: bool = True):
    """load_layer's per-tensor ingest (loader.rs:145-168): GGUF [rows, cols]
    bytes -> f32, transposed to [cols, rows] for 2D weights, sanitized."""
    w = O.dequant(qtype, data, rows * cols).reshape(rows, cols)
    if transpose:
        w = np.ascontiguousarray(w.T)
    return O.sanitize(w)   # sanitize_weights, loader.rs:241-249


class RefEngine:
    """Engine (engine.rs:10-132) over `weights`:
      token_embd, output: GGUF bytes [vocab, d] (output None: tied to the
      embedding); output_norm: f32 [d];
      layers[i]: attn_norm, ffn_norm f32 [d]; attn_q [H*hd, d], attn_k,
      attn_v [KVH*hd, d], attn_o [d, H*hd] GGUF bytes; moe: the MoE layer
      arrays (router, bias, gate, up, down, *_sh) as lco_moe_forward takes."""

    def __init__(self, spec: ModelSpec, weights: dict, threads: int = 8):
        self.s = spec
        self.w = weights
        self.threads = threads
        d, H, KVH, hd, V = spec.d_model, spec.n_head, spec.n_kv_head, spec.head_dim, spec.vocab
        qt = spec.attn_type
        self.embed = ingest(qt, weights["token_embd"], V, d, transpose=False)
        # load_special (loader.rs:193-199): without output.weight the LM head
        # is the embedding transposed
        out = weights.get("output")
        self.lm_head = (np.ascontiguousarray(self.embed.T) if out is None
                        else ingest(qt, out, V, d))                   # [d, V]
        # every f32 tensor load_layer / load_special return is sanitised
        # too (loader.rs:161, :188): the norms here
        self.out_norm = O.sanitize(weights["output_norm"])
        self.layers = []
        for lw in weights["layers"]:
            self.layers.append({
                "wq": ingest(qt, lw["attn_q"], H * hd, d),
                "wk": ingest(qt, lw["attn_k"], KVH * hd, d),
                "wv": ingest(qt, lw["attn_v"], KVH * hd, d),
                "wo": ingest(qt, lw["attn_o"], d, H * hd),
                "attn_norm": O.sanitize(lw["attn_norm"]),
                "ffn_norm": O.sanitize(lw["ffn_norm"]),
            })
        # when set, forward() appends each layer's routing (topk_idx, topk_w
        # of its tokens) to self.routing, in layer order
        self.record_routing = False
        self.routing = []
        self.clear()

    def clear(self):
        """KVCache::clear (cache/mod.rs:27-31)."""
        self.kc = [np.zeros((0, self.s.n_kv_head * self.s.head_dim), np.uint16)
                   for _ in self.layers]
        self.vc = [np.zeros_like(k) for k in self.kc]

    def _mm(self, a, b):
        return O.matmul(a, b, threads=self.threads)

    def forward(self, tokens) -> np.ndarray:
        """Engine::forward (engine.rs:78-132): logits of the last token."""
        s = self.s
        d, H, KVH, hd = s.d_model, s.n_head, s.n_kv_head, s.head_dim
        tokens = list(tokens)
        hidden = np.zeros((len(tokens), d), np.float32)
        for i, t in enumerate(tokens):
            if 0 <= t < s.vocab:
                hidden[i] = self.embed[t]
        for li, (L, lw) in enumerate(zip(self.layers, self.w["layers"])):
            normed = O.rms_norm(hidden, L["attn_norm"], s.eps)
            q = self._mm(normed, L["wq"])
            k = self._mm(normed, L["wk"])
            v = self._mm(normed, L["wv"])
            pos0 = 0 if s.rope_positions == ROPE_PER_CALL else self.kc[li].shape[0]
            q = O.rope(q, H, hd, s.rope_theta, pos0)
            k = O.rope(k, KVH, hd, s.rope_theta, pos0)
            # KVCache::append stores f16 (cache/mod.rs:33-63); get() widens
            self.kc[li] = np.concatenate([self.kc[li], O.f32_to_f16_bits(k)])
            self.vc[li] = np.concatenate([self.vc[li], O.f32_to_f16_bits(v)])
            attn = O.attention_core(q, O.f16_bits_to_f32(self.kc[li]),
                                    O.f16_bits_to_f32(self.vc[li]), H, KVH, hd)
            hidden = hidden + self._mm(attn, L["wo"])
            normed = O.rms_norm(hidden, L["ffn_norm"], s.eps)
            moe = O.moe_forward(s.moe_desc, lw["moe"], normed, threads=self.threads)
            if self.record_routing:
                self.routing.append({"topk_idx": moe["topk_idx"], "topk_w": moe["topk_w"]})
            hidden = hidden + moe["y"]
        hidden = O.rms_norm(hidden, self.out_norm, s.eps)
        return self._mm(hidden[-1:], self.lm_head)[0]

    def generate(self, prompt, n_new: int, eos: int = -1):
        """Engine::generate (engine.rs:51-76) with greedy sampling; stops
        after `eos` when eos >= 0 (the reference stops at id 2)."""
        self.clear()
        logits = self.forward(prompt)
        out = [O.argmax_last(logits)]
        trace = [logits]
        while len(out) < n_new and out[-1] != eos:
            logits = self.forward([out[-1]])
            trace.append(logits)
            out.append(O.argmax_last(logits))
        return out, trace
