"""Pins the oracle's restatement of the engine around the MoE FFN (no GPU):
lco_rope (attention.rs:13-34), lco_attention_core (attention.rs:56-115),
lco_argmax_last (sampler.rs:8-10) and the composition oracle/lcengine.py
(engine.rs:78-132), each against closed forms, special cases and an
independent float64 engine written here with numpy."""
import numpy as np
import pytest

import lcengine as E
import lcoracle as O
import leafcutterllm_amd as L
from leafcutterllm_amd.configs import ModelConfig, small_config, synth_model
from test_oracle_route import layer64


# ------------------------------------------------------------------ rope ---

def test_rope_position_zero_is_identity_and_pairs_are_half_apart():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 4 * 64)).astype(np.float32)
    assert np.array_equal(O.rope(x, 4, 64, 10000.0), x)       # token 0 of a call
    y = np.zeros((2, 2 * 16), np.float32)
    y[1, 3] = 1.0                                              # token 1, head 0, d = 3
    r = O.rope(y, 2, 16, 10000.0)
    nz = np.nonzero(r)
    assert set(nz[1]) == {3, 3 + 8} and set(nz[0]) == {1}      # pair (d, d + hd/2)


def test_rope_angles_vs_float64_and_norms():
    rng = np.random.default_rng(1)
    seq, H, hd, theta = 40, 3, 32, 10000.0
    x = rng.standard_normal((seq, H * hd)).astype(np.float32)
    for pos0 in (0, 500):
        r = O.rope(x, H, hd, theta, pos0).reshape(seq, H, hd).astype(np.float64)
        x3 = x.reshape(seq, H, hd).astype(np.float64)
        pos = (pos0 + np.arange(seq))[:, None, None]
        d = np.arange(hd // 2)[None, None, :]
        ang = pos * theta ** (-2.0 * d / hd)
        x1, x2 = x3[..., :hd // 2], x3[..., hd // 2:]
        e1 = x1 * np.cos(ang) - x2 * np.sin(ang)
        e2 = x1 * np.sin(ang) + x2 * np.cos(ang)
        # the f32 angle carries ~|pos| * 2^-24 of absolute error
        tol = 1e-6 + 4 * (pos0 + seq) * 2.0 ** -24
        assert np.all(np.abs(r[..., :hd // 2] - e1) <= tol * (np.abs(x1) + np.abs(x2)) + 1e-6)
        assert np.all(np.abs(r[..., hd // 2:] - e2) <= tol * (np.abs(x1) + np.abs(x2)) + 1e-6)
        n0 = x1 ** 2 + x2 ** 2
        n1 = r[..., :hd // 2] ** 2 + r[..., hd // 2:] ** 2
        assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------- attention ---

def attention64(q, k, v, H, KVH, hd):
    seq, total = q.shape[0], k.shape[0]
    q = q.reshape(seq, H, hd).astype(np.float64)
    k = k.reshape(total, KVH, hd).astype(np.float64)
    v = v.reshape(total, KVH, hd).astype(np.float64)
    out = np.zeros((seq, H, hd))
    for h in range(H):
        kvh = h // (H // KVH)
        for s in range(seq):
            vis = total - seq + s + 1
            sc = k[:vis, kvh] @ q[s, h] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            out[s, h] = (p / p.sum()) @ v[:vis, kvh]
    return out.reshape(seq, H * hd)


def test_attention_vs_float64_gqa_and_cache():
    rng = np.random.default_rng(2)
    H, KVH, hd, seq, total = 4, 2, 32, 3, 7
    q = rng.standard_normal((seq, H * hd)).astype(np.float32)
    k = rng.standard_normal((total, KVH * hd)).astype(np.float32)
    v = rng.standard_normal((total, KVH * hd)).astype(np.float32)
    out = O.attention_core(q, k, v, H, KVH, hd)
    ref = attention64(q, k, v, H, KVH, hd)
    assert np.max(np.abs(out - ref)) < 1e-5 * np.max(np.abs(ref))
    # heads 0-1 read kv head 0, heads 2-3 kv head 1
    v2 = v.copy()
    v2[:, hd:] += 1.0
    out2 = O.attention_core(q, k, v2, H, KVH, hd)
    assert np.array_equal(out2[:, :2 * hd], out[:, :2 * hd])
    assert not np.array_equal(out2[:, 2 * hd:], out[:, 2 * hd:])


def test_attention_one_key_and_causal_mask():
    rng = np.random.default_rng(3)
    H, hd = 2, 16
    q = rng.standard_normal((1, H * hd)).astype(np.float32)
    k = rng.standard_normal((1, H * hd)).astype(np.float32)
    v = rng.standard_normal((1, H * hd)).astype(np.float32)
    assert np.array_equal(O.attention_core(q, k, v, H, H, hd), v)   # softmax of one score = 1
    seq, total = 4, 6
    q = rng.standard_normal((seq, H * hd)).astype(np.float32)
    k = rng.standard_normal((total, H * hd)).astype(np.float32)
    v = rng.standard_normal((total, H * hd)).astype(np.float32)
    base = O.attention_core(q, k, v, H, H, hd)
    k2, v2 = k.copy(), v.copy()
    k2[4:] += 3.0
    v2[4:] -= 2.0                                 # positions 4, 5: seen by queries 2, 3 only
    other = O.attention_core(q, k2, v2, H, H, hd)
    assert np.array_equal(other[:2], base[:2]) and not np.array_equal(other[2:], base[2:])


# ----------------------------------------------------------------- argmax ---

def test_greedy_argmax_rules():
    f = lambda *v: O.argmax_last(np.array(v, np.float32))
    assert f(0.1, 0.5, 0.3) == 1                  # sampler.rs:57-61
    assert f(1.0, 3.0, 3.0, 2.0) == 2             # the last of equal maxima
    assert f(0.0, -0.0) == 0 and f(-0.0, 0.0) == 1  # total_cmp: -0 < +0
    assert f(1.0, np.nan, 2.0) == 1               # +NaN above +inf
    assert f(-np.inf, -np.inf, -np.inf) == 2
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    assert O.argmax_last(np.array([neg_nan, -np.inf], np.float32)) == 1  # -NaN lowest
    assert O.argmax_last(np.zeros(0, np.float32)) == 0


# ---------------------------------------------------------- the engine ------

TINY = ModelConfig("tiny", 2, 4, 2, 64, 96, 10000.0,
                   small_config("tiny-moe", 256, 256, 8, 2, L.ROUTE_SOFTMAX_RENORM, L.TYPE_Q4_K,
                                L.TYPE_Q4_K, n_shared=1, d_ff_shared=256))


def spec(mc, rope_mode, n_layer=0):
    from parity_util import oracle_desc
    return E.ModelSpec(n_layer or mc.n_layer, mc.d_model, mc.n_head, mc.n_kv_head, mc.head_dim,
                       mc.vocab, mc.rope_theta, mc.attn_type, oracle_desc(mc.layer.desc(64)),
                       rope_positions=rope_mode)


def engine64(s: E.ModelSpec, w: dict, calls):
    """The decoder forward in float64 over the dequantised weights (f16 KV
    storage as the reference); returns the last-token logits per call."""
    d, H, KVH, hd = s.d_model, s.n_head, s.n_kv_head, s.head_dim
    deq = lambda b, r, c: O.dequant(s.attn_type, b, r * c).reshape(r, c).astype(np.float64)
    emb = deq(w["token_embd"], s.vocab, d)
    out_w = deq(w["output"], s.vocab, d)

    def norm(x, g):
        return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + s.eps) * g.astype(np.float64)

    def rope(x, heads, pos):
        x = x.reshape(len(pos), heads, hd).copy()
        ang = np.asarray(pos, np.float64)[:, None, None] * s.rope_theta ** (-2.0 * np.arange(hd // 2) / hd)
        x1, x2 = x[..., :hd // 2].copy(), x[..., hd // 2:].copy()
        x[..., :hd // 2] = x1 * np.cos(ang) - x2 * np.sin(ang)
        x[..., hd // 2:] = x1 * np.sin(ang) + x2 * np.cos(ang)
        return x.reshape(len(pos), heads * hd)

    kc = [np.zeros((0, KVH * hd)) for _ in w["layers"]]
    vc = [np.zeros((0, KVH * hd)) for _ in w["layers"]]
    res = []
    for toks in calls:
        x = np.array([emb[t] if 0 <= t < s.vocab else np.zeros(d) for t in toks])
        for li, lw in enumerate(w["layers"]):
            n = norm(x, lw["attn_norm"])
            q = n @ deq(lw["attn_q"], H * hd, d).T
            k = n @ deq(lw["attn_k"], KVH * hd, d).T
            v = n @ deq(lw["attn_v"], KVH * hd, d).T
            base = 0 if s.rope_positions == E.ROPE_PER_CALL else kc[li].shape[0]
            pos = base + np.arange(len(toks))
            q, k = rope(q, H, pos), rope(k, KVH, pos)
            kc[li] = np.concatenate([kc[li], k.astype(np.float16).astype(np.float64)])
            vc[li] = np.concatenate([vc[li], v.astype(np.float16).astype(np.float64)])
            a = attention64(q, kc[li], vc[li], H, KVH, hd)
            x = x + a @ deq(lw["attn_o"], d, H * hd).T
            y64 = layer64(s.moe_desc, lw["moe"], norm(x, lw["ffn_norm"]).astype(np.float32))[0]
            x = x + y64
        res.append(norm(x[-1:], w["output_norm"]) @ out_w.T)
    return [r[0] for r in res]


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize("mode", [E.ROPE_PER_CALL, E.ROPE_ABSOLUTE])
def test_engine_vs_float64(mode):
    w = synth_model(TINY, seed=3)
    s = spec(TINY, mode)
    eng = E.RefEngine(s, w, threads=4)
    calls = [[5, 17, 3, 95, 0, 60], [11], [200], [42]]   # 200: outside the vocabulary
    got = [eng.forward(c) for c in calls]
    ref = engine64(s, w, calls)
    for g, r in zip(got, ref):
        assert rel(g, r) < 1e-4, rel(g, r)


def test_engine_cache_matches_one_call_with_absolute_positions():
    """With absolute positions, decoding through the KV cache equals one
    forward over the whole sequence; with the reference's per-call
    positions it does not (a decode token is rotated by position 0)."""
    w = synth_model(TINY, seed=4)
    seqs = [7, 8, 9, 10, 11]
    for mode, same in ((E.ROPE_ABSOLUTE, True), (E.ROPE_PER_CALL, False)):
        eng = E.RefEngine(spec(TINY, mode), w, threads=4)
        eng.forward(seqs[:4])
        inc = eng.forward(seqs[4:])
        eng.clear()
        full = eng.forward(seqs)
        assert (rel(inc, full.astype(np.float64)) < 1e-5) == same


def test_engine_generate_is_greedy_over_forward():
    w = synth_model(TINY, seed=5)
    eng = E.RefEngine(spec(TINY, E.ROPE_PER_CALL), w, threads=4)
    toks, trace = eng.generate([1, 2, 3], 5)
    assert len(toks) == 5 and all(t == O.argmax_last(l) for t, l in zip(toks, trace))
    eng2 = E.RefEngine(spec(TINY, E.ROPE_PER_CALL), w, threads=4)
    assert np.array_equal(eng2.forward([1, 2, 3]), trace[0])
    assert np.array_equal(eng2.forward([toks[0]]), trace[1])
    stop, _ = eng.generate([1, 2, 3], 5, eos=toks[1])
    assert stop == toks[:toks.index(toks[1]) + 1]   # up to and including the first eos
