"""GPU: weights that trip the reference's sanitize_weights
(rust/src/model/loader.rs:241-249: NaN, +-Inf and |v| > 100 become 0, for
every tensor load_layer / load_special return) give the oracle's results on
every kernel path.

Planted blocks (their decoded values are exact, so which elements the rule
zeroes is known, tests/test_sanitize_cpu.py):
  * Q8_0 with scale 1 and q = 127 / -101 (zero-coded in place: the
    row-per-lane Q8_0 kernels keep running);
  * Q4_K whose outliers sit in sub-blocks with m = 0 (zero-coded in place:
    the RPL64 row-per-lane and matrix-core kernels keep running);
  * Q4_K whose outliers cannot be zero-coded (the matrix kind is stored as
    sanitised f32 and runs the generic kernels);
  * Q6_K downs with 4q = 104, -128 (zero-coded: row-per-lane and
    matrix-core Q6_K downs);
  * router entries NaN / -inf / 150 and bias entries NaN / 500;
in routed and shared experts.  Bar as every layer test: routing bit-exact
against the oracle, y within 1e-3 relative L2 of the (sanitising) oracle.
"""
import numpy as np
import pytest

import lcengine as E
import leafcutterllm_amd as L
from kquant_pack import pack_q4_k, pack_q6_k, pack_q8_0
from leafcutterllm_amd.configs import ModelConfig, small_config, synth_model, tensor_size
from parity_util import run_and_check
from test_oracle_engine import rel, spec

pytestmark = pytest.mark.gpu

Q4, Q6, Q8 = L.TYPE_Q4_K, L.TYPE_Q6_K, L.TYPE_Q8_0


def blk_q8():
    q = [0] * 32
    q[3], q[10], q[20], q[31] = 127, -101, 100, 9
    return pack_q8_0(1.0, q)


def blk_q4_zeroable(rng):
    """m = 0 everywhere: q = 0 decodes to 0, q >= 1 to 63 q >= 63 (q >= 2: out)."""
    return pack_q4_k(1.0, 0.5, [63] * 8, [0] * 8, rng.integers(0, 3, 256))


def blk_q4_unzeroable(rng):
    """dmin * m = 0.01: q = 0 decodes to -0.01, q >= 1 to >= 125.99 (out)."""
    return pack_q4_k(2.0, 0.01, [63] * 8, [1] * 8, rng.integers(0, 2, 256))


def blk_q6(rng):
    q = rng.integers(-3, 4, 256)
    q[::17] = 26   # 4 * 26 = 104
    q[::29] = -32  # -128
    return pack_q6_k(1.0, [4] * 16, q)


def plant(arr, qt, rows, cols, n_mats, blob, every=5):
    """Overwrites every `every`-th block of each of the n_mats stacked
    [rows, cols] matrices with `blob` (one block of qt) -- a copy."""
    out = arr.copy()
    bb, bs = len(blob), (32 if qt == Q8 else 256)
    sz = tensor_size(qt, rows * cols)
    nb = rows * cols // bs
    for m in range(n_mats):
        for b in range(m % every, nb, every):
            out[m * sz + b * bb: m * sz + (b + 1) * bb] = np.frombuffer(blob, np.uint8)
    return out


def outliers(qt, arr, n):
    _, z, u = L.sanitize_blocks(qt, arr, n)
    return z + u


def dirty_router(layer, E_):
    r = layer["router"].copy()
    r[1, 0], r[7, E_ - 1], r[30, E_ // 2] = np.nan, -np.inf, 150.0
    return r


def test_q8_outliers_row_per_lane_with_shared():
    cfg = small_config("san-q8", 512, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q8, Q8, n_shared=1,
                       d_ff_shared=512)
    layer = L.synth_layer(cfg, seed=21)
    b = blk_q8()
    for k, rows, cols, n in (("gate", 512, 512, 8), ("up", 512, 512, 8), ("down", 512, 512, 8),
                             ("gate_sh", 512, 512, 1), ("down_sh", 512, 512, 1)):
        layer[k] = plant(layer[k], Q8, rows, cols, n, b)
    assert outliers(Q8, layer["gate"], 512 * 512 * 8) > 0
    layer["router"] = dirty_router(layer, 8)
    for T in (1, 5, 40):
        x = L.synth_x(cfg, T, seed=21, index=T)
        print(f"sanitize q8 T={T}", flush=True)
        run_and_check(cfg, layer, x)


@pytest.mark.parametrize("kind", ["zeroable", "f32"])
def test_q4k_outliers(kind):
    """Zero-codable outliers keep the RPL64 kernels (row-per-lane at T = 2,
    matrix cores at T = 48); the others move the matrix kind to f32."""
    cfg = small_config("san-q4", 512, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4, n_shared=1,
                       d_ff_shared=512)
    layer = L.synth_layer(cfg, seed=22)
    rng = np.random.default_rng(22)
    mk = blk_q4_zeroable if kind == "zeroable" else blk_q4_unzeroable
    layer["up"] = plant(layer["up"], Q4, 512, 512, 8, mk(rng))
    layer["down"] = plant(layer["down"], Q4, 512, 512, 8, mk(rng), every=7)
    layer["up_sh"] = plant(layer["up_sh"], Q4, 512, 512, 1, mk(rng))
    _, z, u = L.sanitize_blocks(Q4, layer["up"], 512 * 512 * 8)
    assert (u == 0 and z > 0) if kind == "zeroable" else u > 0
    for T in (2, 48):
        x = L.synth_x(cfg, T, seed=22, index=T)
        print(f"sanitize q4 {kind} T={T}", flush=True)
        run_and_check(cfg, layer, x)


def test_q6k_down_outliers_sigmoid_group():
    """Config-4 semantics at a small shape: Q6_K downs with outliers (row-per-
    lane at T = 1, 8; matrix cores at T = 64), zero-codable Q4_K gates, a
    bias with NaN and 500, a dirty router."""
    cfg = small_config("san-q6", 512, 512, 32, 4, L.ROUTE_SIGMOID_GROUP, Q4, Q6, n_group=4,
                       topk_group=2, routed_scale=2.5, bias="normal0.1", n_shared=1,
                       d_ff_shared=512)
    layer = L.synth_layer(cfg, seed=23)
    rng = np.random.default_rng(23)
    layer["down"] = plant(layer["down"], Q6, 512, 512, 32, blk_q6(rng))
    layer["down_sh"] = plant(layer["down_sh"], Q6, 512, 512, 1, blk_q6(rng))
    layer["gate"] = plant(layer["gate"], Q4, 512, 512, 32, blk_q4_zeroable(rng), every=9)
    assert outliers(Q6, layer["down"], 512 * 512 * 32) > 0
    bias = layer["bias"].copy()
    bias[3], bias[17] = np.nan, 500.0
    layer["bias"] = bias
    layer["router"] = dirty_router(layer, 32)
    for T in (1, 8, 64):
        x = L.synth_x(cfg, T, seed=23, index=T)
        print(f"sanitize q6 T={T}", flush=True)
        run_and_check(cfg, layer, x)


def test_norm_residual_sanitizes_norm_weight():
    """lcmoe_set_norm sanitises the post-attention norm weight."""
    import lcoracle as O
    from parity_util import oracle_desc
    cfg = small_config("san-norm", 512, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4)
    layer = L.synth_layer(cfg, seed=24)
    w = (1.0 + L.configs.synth_normal(24, 3, 0.02, 512)).astype(np.float32)
    w[[0, 100, 300, 511]] = [np.nan, 1e3, -np.inf, -100.0]
    hidden = L.synth_x(cfg, 6, seed=24, index=1)
    with L.MoeFfn(cfg.desc(8), layer) as moe:
        moe.set_norm(w, 1e-5)
        out = moe.forward_norm_residual(hidden)[0]
    normed = O.rms_norm(hidden, O.sanitize(w), 1e-5)
    ref = hidden + O.moe_forward(oracle_desc(cfg.desc(8)), layer, normed)["y"]
    assert np.all(np.isfinite(out))
    assert rel(out, ref.astype(np.float64)) < 1e-3


def test_model_sanitizes_every_tensor_and_ties_the_head():
    """A tiny model whose attention projections, embedding and norms hold
    outliers (q/k/v with blocks Q4_K cannot zero -> f32; o zero-codable),
    with no output tensor (the LM head tied to the embedding)."""
    mc = ModelConfig("tiny-san", 2, 4, 2, 64, 96, 10000.0,
                     small_config("tiny-san-moe", 256, 256, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4,
                                  n_shared=1, d_ff_shared=256))
    w = synth_model(mc, seed=25)
    rng = np.random.default_rng(25)
    d, qd = 256, 4 * 64
    w["token_embd"] = plant(w["token_embd"], Q4, 96, d, 1, blk_q4_unzeroable(rng), every=11)
    w.pop("output")
    for l, lw in enumerate(w["layers"]):
        lw["attn_k"] = plant(lw["attn_k"], Q4, 2 * 64, d, 1, blk_q4_unzeroable(rng), every=13)
        lw["attn_o"] = plant(lw["attn_o"], Q4, d, qd, 1, blk_q4_zeroable(rng), every=9)
        for k in ("attn_norm", "ffn_norm"):
            lw[k] = lw[k].copy()
            lw[k][[l, 50 + l, 200]] = [np.nan, 250.0, -np.inf]
    w["output_norm"] = w["output_norm"].copy()
    w["output_norm"][7] = np.inf
    ref = E.RefEngine(spec(mc, E.ROPE_ABSOLUTE), w, threads=8)
    with L.Model(mc.desc(2, 16, 64, E.ROPE_ABSOLUTE), w) as m:
        for c in ([5, 17, 3, 95, 0, 60, 20], [11], [42]):
            g = m.forward(np.array([c]))[0]
            r = ref.forward(c).astype(np.float64)
            assert np.all(np.isfinite(g))
            assert rel(g, r) < 1e-3, rel(g, r)


def test_model_refuses_after_a_failed_call_until_reset():
    """A generate whose second internal forward fails (forced from the host:
    the first sequence's prefill has advanced its device cache length) leaves
    the model refusing forward until reset; after the reset it matches a
    fresh model."""
    from test_oracle_engine import TINY
    w = synth_model(TINY, seed=26)
    prompts = np.array([[3, 1, 4, 1, 5], [2, 7, 1, 8, 2]])
    with L.Model(TINY.desc(2, 8, 16, E.ROPE_ABSOLUTE), w) as fresh:
        want, _ = fresh.generate(prompts, 6)
        want_fwd = fresh.forward(np.array([[1], [2]]))
    with L.Model(TINY.desc(2, 8, 16, E.ROPE_ABSOLUTE), w) as m:
        m.debug_fail_forward(1)
        with pytest.raises(L.LcmoeError) as e:
            m.generate(prompts, 6)
        assert "debug_fail_forward" in str(e.value)
        with pytest.raises(L.LcmoeError) as e:
            m.forward(np.array([[1] * 8]))   # would overrun sequence 0's cache
        assert e.value.status == 6  # LCMOE_ERR_STATE
        m.reset()
        got, _ = m.generate(prompts, 6)       # generate resets by itself too
        assert np.array_equal(got, want)
        assert np.array_equal(m.forward(np.array([[1], [2]])), want_fwd)
