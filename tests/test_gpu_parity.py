"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bar: topk_idx / counts / offsets / perm / inv bit-identical; routed weights
within 1e-5 relative; layer output within 1e-3 relative L2 over [T, d];
device decoders and the router sigmoid bit-identical to the oracle.
"""
import numpy as np
import pytest

import lcoracle as O
import leafcutterllm_amd as L
from kquant_pack import pack_q4_k, pack_q6_k, pack_q8_0
from leafcutterllm_amd.configs import small_config
from parity_util import oracle_desc, rel_l2, run_and_check

pytestmark = pytest.mark.gpu

Q4, Q6, Q8 = L.TYPE_Q4_K, L.TYPE_Q6_K, L.TYPE_Q8_0


def u8(b):
    return np.frombuffer(b, np.uint8).copy()


# ----------------------------------------------------------- decoders ------

@pytest.mark.parametrize("qtype", [Q8, Q4, Q6])
def test_device_decoder_bit_exact(qtype):
    x = L.configs.synth_normal(3, 9, 0.02, 256 * 96)
    x[:256] *= 1e-6   # tiny scales: f16 subnormal d
    x[256:512] *= 300.0
    data = L.configs.quantize(qtype, x)
    dev = L.debug_dequant(qtype, data, x.size)
    ref = O.dequant(qtype, data, x.size)
    assert np.array_equal(dev.view(np.uint32), ref.view(np.uint32))


def test_device_decoder_hand_built_blocks():
    rng = np.random.default_rng(5)
    q4 = b"".join(pack_q4_k(float(d), float(m), rng.integers(0, 64, 8), rng.integers(0, 64, 8),
                            rng.integers(0, 16, 256))
                  for d, m in [(1.0, 0.5), (6e-8, 3e-5), (0.01, 0.0), (-0.25, -1.0)])
    q6 = b"".join(pack_q6_k(float(d), rng.integers(-128, 128, 16), rng.integers(-32, 32, 256))
                  for d in [1.0, 6e-8, -0.5])
    q8 = b"".join(pack_q8_0(float(d), rng.integers(-128, 128, 32)) for d in [0.5, -3e-6, 100.0])
    for qt, blob, n in [(Q4, q4, 4 * 256), (Q6, q6, 3 * 256), (Q8, q8, 3 * 32)]:
        dev = L.debug_dequant(qt, u8(blob), n)
        ref = O.dequant(qt, u8(blob), n)
        assert np.array_equal(dev.view(np.uint32), ref.view(np.uint32)), qt


def test_device_sigmoid_bit_exact():
    x = np.concatenate([np.linspace(-110, 110, 150001, dtype=np.float32),
                        np.linspace(-1, 1, 50001, dtype=np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, 88.7, -88.7, 1e-30], np.float32)])
    dev = L.debug_sigmoid(x)
    ref = O.sigmoid_cw(x)
    assert np.array_equal(dev.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------- small layers ------

SMALL = {
    "q4k-renorm": small_config("q4k-renorm", 256, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4),
    "q8-renorm": small_config("q8-renorm", 256, 384, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q8, Q8),
    "q4k-straddle-shared-bias": small_config(
        "q4k-straddle", 256, 352, 12, 3, L.ROUTE_SOFTMAX, Q4, Q4, n_shared=2, d_ff_shared=352,
        bias="plus2_first8"),
    "sigmoid-group-q6k": small_config(
        "sig", 512, 256, 32, 4, L.ROUTE_SIGMOID_GROUP, Q4, Q6, n_shared=1, d_ff_shared=256,
        n_group=4, topk_group=2, routed_scale=2.5, bias="normal0.1"),
    "e60-tail": small_config("e60", 256, 256, 60, 4, L.ROUTE_SOFTMAX, Q4, Q4),
    "q6k-all": small_config("q6", 512, 512, 16, 8, L.ROUTE_SOFTMAX_RENORM, Q6, Q6),
    "f32": small_config("f32", 128, 256, 4, 2, L.ROUTE_SOFTMAX_RENORM, L.TYPE_F32, L.TYPE_F32),
    # d_ff an odd multiple of 128: Q4_K down blocks straddle rows (split layout)
    "q4k-split-shared": small_config(
        "split", 256, 384, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4, n_shared=2, d_ff_shared=640),
    # Q8_0 everywhere in the row-per-lane layout, with a fused shared expert
    "q8-rpl-shared": small_config(
        "q8rpl", 256, 512, 8, 2, L.ROUTE_SOFTMAX, Q8, Q8, n_shared=1, d_ff_shared=512),
    # Q6_K down with a 4-way column split and 4 shared experts
    "q6k-down-e16": small_config(
        "q6dn", 512, 1024, 16, 4, L.ROUTE_SOFTMAX, Q4, Q6, n_shared=1, d_ff_shared=512),
    # d_model not a multiple of 256 (nor 128): K-quant blocks straddle rows of
    # gate/up, generic expert kernels and the exact router
    "q4k-d288-generic": small_config(
        "d288", 288, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4, n_shared=1, d_ff_shared=256),
    # more than 8 experts per token: the combine's loop form
    "k12-shared": small_config(
        "k12", 256, 256, 32, 12, L.ROUTE_SOFTMAX_RENORM, Q4, Q4, n_shared=1, d_ff_shared=256),
    # E % 8 == 4 past 64 experts: at T * E * d > 2^25 the chain router's
    # streaming logits product, with its own block of tail columns
    "e68-chain": small_config("e68", 512, 256, 68, 4, L.ROUTE_SOFTMAX, Q4, Q4),
    "sig64-chain": small_config(
        "sig64", 512, 256, 64, 4, L.ROUTE_SIGMOID_GROUP, Q4, Q6, n_group=8, topk_group=4,
        routed_scale=2.5, bias="normal0.1"),
}


@pytest.mark.parametrize("name", sorted(SMALL))
@pytest.mark.parametrize("T", [1, 3, 8, 17, 64])
def test_small_layer_parity(name, T):
    cfg = SMALL[name]
    layer = L.synth_layer(cfg, seed=11)
    x = L.synth_x(cfg, T, seed=11, index=T)
    res = run_and_check(cfg, layer, x)
    assert res["rel_l2"] < 1e-3


@pytest.mark.parametrize("name,T", [("q6k-down-e16", 160), ("q4k-split-shared", 200),
                                    ("sigmoid-group-q6k", 300), ("e68-chain", 1000),
                                    ("sig64-chain", 1100)])
def test_small_layer_parity_many_tokens(name, T):
    """Tens of tokens per expert: 32-token matrix-core passes (Q6_K, split
    Q4_K), several pass groups per slot and prefill-style shared launches;
    the last two run the chain router (exact logits of every token and
    expert, T * E * d > 2^25)."""
    cfg = SMALL[name]
    layer = L.synth_layer(cfg, seed=5)
    x = L.synth_x(cfg, T, seed=5, index=T)
    res = run_and_check(cfg, layer, x)
    assert res["rel_l2"] < 1e-3


def test_handle_reuse_and_determinism():
    cfg = SMALL["sigmoid-group-q6k"]
    layer = L.synth_layer(cfg, seed=2)
    with L.MoeFfn(cfg.desc(64), layer) as moe:
        for T in (64, 5, 1, 64, 0, 33):
            x = L.synth_x(cfg, T, seed=2, index=100 + T)
            if T == 0:
                y, idx, w = moe.forward(x.reshape(0, cfg.d_model))
                assert y.shape == (0, cfg.d_model)
                continue
            r1 = run_and_check(cfg, layer, x, moe=moe)
            y2, idx2, _ = moe.forward(x)
            assert np.array_equal(r1["y"], y2)          # run-to-run bit identical
            assert np.array_equal(r1["topk_idx"], idx2)


def test_adversarial_router_ties():
    """Equal logits, +-0, -inf and NaN inputs: ties go to the lower expert."""
    cfg = small_config("ties", 256, 256, 16, 4, L.ROUTE_SOFTMAX_RENORM, Q4, Q4)
    layer = L.synth_layer(cfg, seed=4)
    r = np.zeros((256, 16), np.float32)
    r[0, :] = 1.0          # x[:,0] drives all logits equally
    r[1, 3] = r[1, 9] = 1.0
    layer["router"] = r
    x = np.zeros((8, 256), np.float32)
    x[0, 0] = 1.0                    # all equal -> experts 0..3
    x[1, 1] = 2.0                    # 3 and 9 lead, then ties -> 0, 1
    x[2, 0] = -0.0                   # all zero
    x[3, 0] = np.inf                 # all +inf, ties -> 0..3
    x[4, 0] = -np.inf                # all -inf
    x[5, 0] = np.nan                 # all NaN -> ranks as -inf, 0..3
    x[6, 0], x[6, 1] = 1.0, -1.0     # logits 1 except 3, 9 at 0
    x[7, 1] = 1e-30
    moe = L.MoeFfn(cfg.desc(8), layer)
    try:
        _, idx, _ = moe.forward(x)
        od = oracle_desc(cfg.desc(8))
        with np.errstate(all="ignore"):
            r_idx, _ = O.route(od, O.router_logits(x, r))
        assert np.array_equal(idx, r_idx)
        assert list(idx[0]) == [0, 1, 2, 3] and list(idx[1]) == [3, 9, 0, 1]
        disp = moe.dispatch()
        counts, offsets, perm, inv = O.dispatch(r_idx, 16)
        assert np.array_equal(disp["perm"], perm) and np.array_equal(disp["inv"], inv)
    finally:
        moe.close()


# d = 1024: the exact router chains are split by column between the router
# launch and the gate/up launch on the row-per-lane path (T <= 3 here) and run
# whole in the matrix-core gate/up launch (T >= 4)
CHAIN_CFG = small_config("chains", 1024, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q4, Q4)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 16, 40])
def test_router_chain_split_parity(T):
    layer = L.synth_layer(CHAIN_CFG, seed=21)
    x = L.synth_x(CHAIN_CFG, T, seed=21, index=T)
    res = run_and_check(CHAIN_CFG, layer, x)
    assert res["rel_l2"] < 1e-3


# E = 12: a partial second chain tile (experts 8..11 on the mul+add tail)
CHAIN_CFG12 = small_config("chains12", 1024, 256, 12, 3, L.ROUTE_SOFTMAX, Q4, Q4, n_shared=1,
                           d_ff_shared=256)


@pytest.mark.parametrize("T", [1, 2, 9, 33])
def test_router_chain_split_partial_tiles(T):
    layer = L.synth_layer(CHAIN_CFG12, seed=23)
    x = L.synth_x(CHAIN_CFG12, T, seed=23, index=T)
    res = run_and_check(CHAIN_CFG12, layer, x)
    assert res["rel_l2"] < 1e-3


@pytest.mark.parametrize("T", [1, 2, 3, 4, 16])
def test_router_fallback_with_chain_split(T):
    """Experts 0 and 1 share one router row, so their scores tie exactly and
    the certified router cannot order them: every token that ranks them near
    the top-k boundary takes the exact fallback (ties to the lower index),
    while the column-split chains still produce the routing weights."""
    layer = L.synth_layer(CHAIN_CFG, seed=22)
    r = layer["router"].copy()
    r[:, 1] = r[:, 0]
    layer["router"] = r
    x = L.synth_x(CHAIN_CFG, T, seed=22, index=T)
    res = run_and_check(CHAIN_CFG, layer, x)
    assert res["rel_l2"] < 1e-3
    idx = res["topk_idx"].reshape(T, 2)
    both = np.sum((idx == 0).any(axis=1) & (idx == 1).any(axis=1))
    if both:  # a token holding both tied experts ranks 0 before 1
        rows = (idx == 0).any(axis=1) & (idx == 1).any(axis=1)
        assert np.all(np.argmax(idx[rows] == 0, axis=1) < np.argmax(idx[rows] == 1, axis=1))


# ------------------------------------------ certified sigmoid-group router --

SIG_CFG = small_config("sig64", 512, 256, 64, 8, L.ROUTE_SIGMOID_GROUP, Q4, Q6, n_shared=1,
                       d_ff_shared=256, n_group=8, topk_group=4, routed_scale=2.5,
                       bias="normal0.1")


@pytest.mark.parametrize("T", [1, 5, 32, 100])
def test_sigmoid_certified_router(T):
    """float64 bounds settle the group and expert selection of (nearly) every
    token; routing, dispatch and weights equal the oracle's exact chains."""
    layer = L.synth_layer(SIG_CFG, seed=31)
    x = L.synth_x(SIG_CFG, T, seed=31, index=T)
    with L.MoeFfn(SIG_CFG.desc(T), layer) as moe:
        res = run_and_check(SIG_CFG, layer, x, moe=moe)
        fb = moe.route_fallbacks()
    assert res["rel_l2"] < 1e-3
    assert 0 <= fb <= max(1, T // 8), fb


@pytest.mark.parametrize("T", [1, 7, 40])
def test_sigmoid_router_exact_ties_fall_back(T):
    """Experts 0 and 1 (group 0) share a router row and a +1 bias: their keys
    tie exactly and lead every token, so no float64 bound can order them and
    every token takes the exact chains, which rank 0 before 1."""
    layer = L.synth_layer(SIG_CFG, seed=32)
    r = layer["router"].copy()
    r[:, 1] = r[:, 0]
    layer["router"] = r
    b = layer["bias"].copy()
    b[0] = b[1] = 1.0
    layer["bias"] = b
    x = L.synth_x(SIG_CFG, T, seed=32, index=T)
    with L.MoeFfn(SIG_CFG.desc(T), layer) as moe:
        res = run_and_check(SIG_CFG, layer, x, moe=moe)
        assert moe.route_fallbacks() == T
    idx = res["topk_idx"].reshape(T, SIG_CFG.n_expert_used)
    assert np.all(idx[:, 0] == 0) and np.all(idx[:, 1] == 1)


def test_sigmoid_router_mixed_tokens():
    """Every third token is the one-hot x = e_0, whose logits are row 0 of
    the router: experts 0 and 1 share the top logit 50 and the bias, an exact
    tie for the exact chains to settle; the other tokens (x[0] = 0) certify.
    The chain and select launches serve exactly the marked tokens, and every
    token is dispatched."""
    T = 24
    layer = L.synth_layer(SIG_CFG, seed=33)
    r = layer["router"].copy()
    r[0, :2] = 50.0
    layer["router"] = r
    b = layer["bias"].copy()
    b[1] = b[0]
    layer["bias"] = b
    x = L.synth_x(SIG_CFG, T, seed=33, index=T)
    x[:, 0] = 0.0
    tied = np.arange(T) % 3 == 0
    x[tied] = 0.0
    x[tied, 0] = 1.0
    with L.MoeFfn(SIG_CFG.desc(T), layer) as moe:
        res = run_and_check(SIG_CFG, layer, x, moe=moe)
        fb = moe.route_fallbacks()
    idx = res["topk_idx"].reshape(T, SIG_CFG.n_expert_used)
    assert np.all(idx[tied, 0] == 0) and np.all(idx[tied, 1] == 1)
    assert int(tied.sum()) <= fb <= int(tied.sum()) + max(1, T // 8), fb


# group sizes E / n_group of the certifying wave's butterfly (1 .. 64 lanes,
# aligned blocks of each 64-expert slice) and one it leaves to the LDS path
# (12, not a power of two)
SIG_GROUPS = [(256, 4, 2, 8), (64, 4, 2, 6), (32, 8, 4, 4), (16, 8, 4, 4), (16, 16, 8, 4),
              (48, 4, 2, 6)]


@pytest.mark.parametrize("E,G,TG,K", SIG_GROUPS)
@pytest.mark.parametrize("T", [1, 5])
def test_sigmoid_router_group_sizes(E, G, TG, K, T):
    """The certified sigmoid-group router at group sizes 64, 16, 4, 2, 1 and
    12: routing, dispatch and weights equal the oracle's exact chains."""
    cfg = small_config(f"sig{E}g{G}", 512, 256, E, K, L.ROUTE_SIGMOID_GROUP, Q4, Q6,
                       n_group=G, topk_group=TG, routed_scale=2.5, bias="normal0.1")
    layer = L.synth_layer(cfg, seed=34 + E + G)
    x = L.synth_x(cfg, T, seed=34, index=T)
    with L.MoeFfn(cfg.desc(T), layer) as moe:
        res = run_and_check(cfg, layer, x, moe=moe)
        fb = moe.route_fallbacks()
    assert res["rel_l2"] < 1e-3
    assert 0 <= fb <= max(1, T // 4), fb


@pytest.mark.parametrize("T", [1, 6])
def test_sigmoid_router_group_tie_falls_back(T):
    """Groups 0 and 1 are copies (router columns and biases) that lead every
    token, and only one group is kept: their group scores tie exactly, so no
    bound separates them and every token takes the exact chains, which keep
    the lower group."""
    cfg = small_config("sig32g4", 512, 256, 32, 4, L.ROUTE_SIGMOID_GROUP, Q4, Q6, n_group=4,
                       topk_group=1, routed_scale=2.5, bias="normal0.1")
    layer = L.synth_layer(cfg, seed=35)
    r = layer["router"].copy()
    r[:, 8:16] = r[:, 0:8]
    layer["router"] = r
    b = layer["bias"].copy()
    b[0:8] = 1.0 + 0.01 * np.arange(8)
    b[8:16] = b[0:8]
    layer["bias"] = b
    x = L.synth_x(cfg, T, seed=35, index=T)
    with L.MoeFfn(cfg.desc(T), layer) as moe:
        res = run_and_check(cfg, layer, x, moe=moe)
        assert moe.route_fallbacks() == T
    idx = res["topk_idx"].reshape(T, cfg.n_expert_used)
    assert np.all(idx < 8), idx


WIDE_CFG = small_config("wide64", 512, 256, 64, 4, L.ROUTE_SOFTMAX_RENORM, Q4, Q4, n_shared=1,
                        d_ff_shared=256)


@pytest.mark.parametrize("kind", [L.ROUTE_SOFTMAX_RENORM, L.ROUTE_SOFTMAX])
def test_wide_softmax_router_one_token(kind):
    """E >= 32 at one token: the softmax kinds take the parallel-bounds
    certified router, which certifies (nearly) every token and, in the same
    launch, dispatches; routing, dispatch and weights equal the oracle's."""
    cfg = small_config("wide64", 512, 256, 64, 4, kind, Q4, Q4, n_shared=1, d_ff_shared=256)
    layer = L.synth_layer(cfg, seed=41)
    for i in range(6):
        x = L.synth_x(cfg, 1, seed=41, index=i)
        with L.MoeFfn(cfg.desc(1), layer) as moe:
            res = run_and_check(cfg, layer, x, moe=moe)
            assert 0 <= moe.route_fallbacks() <= 1
        assert res["rel_l2"] < 1e-3


def test_wide_softmax_router_exact_tie_falls_back():
    """Experts 5 and 9 share a router row that leads every logit: their
    bounds cannot order them, so the certifying block runs the exact chains
    and selection itself (one token), which rank 5 before 9."""
    cfg = WIDE_CFG
    layer = L.synth_layer(cfg, seed=43)
    x = L.synth_x(cfg, 1, seed=43, index=0)
    r = layer["router"].copy()
    r[:, 5] = 4.0 * np.sign(x[0]) / np.sqrt(cfg.d_model)
    r[:, 9] = r[:, 5]
    layer["router"] = r
    with L.MoeFfn(cfg.desc(1), layer) as moe:
        res = run_and_check(cfg, layer, x, moe=moe)
        assert moe.route_fallbacks() == 1
    idx = res["topk_idx"].reshape(1, cfg.n_expert_used)
    assert idx[0, 0] == 5 and idx[0, 1] == 9
    assert res["rel_l2"] < 1e-3


@pytest.mark.parametrize("E,T", [(40, 3), (40, 16), (64, 5), (40, 300)])
def test_fast_router_multi_tile_fallback(E, T):
    """More than 8 experts at several tokens (the per-token fast router):
    experts 5 and 9 share a router row that leads every token's logits (all
    token rows carry token 0's sign pattern), so no token can be certified
    and each block runs its token's exact chains, its tiles of 8 experts
    spread over four waves (E = 40: five tiles, so one wave runs two; E =
    64: eight, two per wave; past 256 tokens one wave runs them all, as at
    E <= 8).  Identical rows give identical bounds, which
    never order the pair, so every token takes the fallback; the selection
    ranks 5 before 9 for every token."""
    cfg = small_config(f"fb{E}", 512, 256, E, 4, L.ROUTE_SOFTMAX_RENORM, Q4, Q4)
    layer = L.synth_layer(cfg, seed=47)
    x = L.synth_x(cfg, T, seed=47, index=T)
    x = (np.abs(x) * np.sign(x[0])[None, :]).astype(np.float32)
    r = layer["router"].copy()
    r[:, 5] = 4.0 * np.sign(x[0]) / np.sqrt(cfg.d_model)
    r[:, 9] = r[:, 5]
    layer["router"] = r
    res = run_and_check(cfg, layer, x)
    idx = res["topk_idx"].reshape(T, cfg.n_expert_used)
    assert np.all(idx[:, 0] == 5) and np.all(idx[:, 1] == 9)
    assert res["rel_l2"] < 1e-3


@pytest.mark.parametrize("T", [3, 16, 64])
def test_q8_large_weights_h_beyond_f16(T):
    """Q8_0 experts whose every block has scale 1 and |q| <= 100 (the largest
    weights the loader keeps): gate and up sums reach ~1e3 and H ~1e6, far
    past the f16 range.  The matrix-core path (T * K > E) carries H as f16
    scaled by a power of two per token and 32-column block; the row-per-lane
    path (T = 3) as int8 limbs.  Both stay within the layer bar."""
    cfg = small_config("q8big", 512, 512, 8, 2, L.ROUTE_SOFTMAX_RENORM, Q8, Q8, n_shared=1,
                       d_ff_shared=512)
    layer = L.synth_layer(cfg, seed=53)
    rng = np.random.default_rng(53)
    for k, n in (("gate", 8), ("up", 8), ("down", 8), ("gate_sh", 1), ("up_sh", 1),
                 ("down_sh", 1)):
        nb = layer[k].size // 34
        q = rng.integers(-100, 101, (nb, 32))
        blocks = np.zeros((nb, 34), np.uint8)
        blocks[:, :2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        blocks[:, 2:] = q.astype(np.int8).view(np.uint8)
        layer[k] = blocks.reshape(-1)
    x = L.synth_x(cfg, T, seed=53, index=T)
    res = run_and_check(cfg, layer, x)
    assert np.all(np.isfinite(res["y"]))
    assert res["rel_l2"] < 1e-3


def test_e1_k1_reduces_to_dense_ffn():
    """E = 1, K = 1, renormalised: weight exactly 1.0 and the layer is the
    dense SwiGLU ffn_forward (engine.rs:146-164) of the one expert."""
    cfg = small_config("dense", 256, 512, 1, 1, L.ROUTE_SOFTMAX_RENORM, Q4, Q4)
    layer = L.synth_layer(cfg, seed=8)
    x = L.synth_x(cfg, 9, seed=8)
    wg = O.dequant(Q4, layer["gate"], 512 * 256).reshape(512, 256).T
    wu = O.dequant(Q4, layer["up"], 512 * 256).reshape(512, 256).T
    wd = O.dequant(Q4, layer["down"], 256 * 512).reshape(256, 512).T
    with L.MoeFfn(cfg.desc(9), layer) as moe:
        # T = 1: the row-per-lane path: x and H enter the integer products as
        # 15-bit two-limb values (|error| <= max|v| / 32512 per 32-element
        # sub-block), about 1e-4 relative on y
        y, idx, w = moe.forward(x[:1])
        assert idx[0, 0] == 0 and w[0, 0] == 1.0
        assert rel_l2(y, O.ffn_dense(x[:1], wg, wu, wd)) < 2e-4
        # T = 9 > E: the matrix-core path; x as two f16 (about 3e-6), then
        # as one f16 (the default, about 3e-4; the layer bar is 1e-3)
        ref = O.ffn_dense(x, wg, wu, wd)
        moe.set_act_precision(L.ACT_F16X2)
        y, idx, w = moe.forward(x)
        assert np.all(idx == 0) and np.all(w == 1.0)
        assert rel_l2(y, ref) < 2e-5
        moe.set_act_precision(L.ACT_F16)
        y, _, _ = moe.forward(x)
        assert rel_l2(y, ref) < 1e-3


# ------------------------------------------------- full BASELINE shapes -----

FULL_T = [(1, 1), (1, 16), (2, 1), (2, 2), (2, 3), (2, 4), (2, 8), (2, 17), (2, 64), (5, 1),
          (5, 16)]


@pytest.fixture(scope="module")
def full_layers():
    cache = {}

    def get(c):
        if c not in cache:
            cache.clear()
            cfg = L.CONFIGS[c]
            layer = L.synth_layer(cfg, seed=0)
            cache[c] = (cfg, layer, L.MoeFfn(cfg.desc(max(cfg.tokens + (64,))), layer))
        return cache[c]
    yield get
    for v in cache.values():
        v[2].close()


@pytest.mark.parametrize("c,T", FULL_T)
def test_full_config_parity(full_layers, c, T):
    cfg, layer, moe = full_layers(c)
    x = L.synth_x(cfg, T, seed=0, index=T)
    res = run_and_check(cfg, layer, x, moe=moe)
    print(f"config {c} T={T}: rel_l2={res['rel_l2']:.2e} touched={int((res['counts'] > 0).sum())}")


@pytest.mark.parametrize("T", [1, 4, 32, 256])
def test_full_config4_parity(full_layers, T):
    """DeepSeek-V3 shape: sigmoid-group router over 256 experts, Q6_K down
    (matrix-core Q6_K path), one shared expert."""
    cfg, layer, moe = full_layers(4)
    x = L.synth_x(cfg, T, seed=0, index=T)
    res = run_and_check(cfg, layer, x, moe=moe)
    fb = moe.route_fallbacks()
    # decode batches route through the certified sigmoid-group router (T * E
    # * d within its limit), larger ones through the exact chains alone
    assert fb == -1 if T > 18 else 0 <= fb <= max(1, T // 8), fb
    print(f"config 4 T={T}: rel_l2={res['rel_l2']:.2e} touched={int((res['counts'] > 0).sum())} "
          f"uncertified={fb}")


def test_full_config3_prefill_parity(full_layers):
    cfg, layer, moe = full_layers(3)
    x = L.synth_x(cfg, 2048, seed=0, index=2048)
    res = run_and_check(cfg, layer, x, moe=moe)
    counts = res["counts"]
    assert counts[:8].sum() > counts[8:].sum()   # the +2.0 bias skews routing
    print(f"config 3 T=2048: rel_l2={res['rel_l2']:.2e} biased-share={counts[:8].sum() / counts.sum():.2f}")


@pytest.mark.parametrize("c,T", [(2, 64), (3, 256), (4, 256)])
def test_activation_precision_modes(full_layers, c, T):
    """The matrix-core gate/up products in both activation modes on the
    same inputs: LCMOE_ACT_F16 (the default, one f16 per element) within the
    1e-3 bar, LCMOE_ACT_F16X2 (two f16) within 2e-5 -- and the two differ,
    so the mode reaches the kernel.  Routing is bit-exact in both (it does
    not depend on the mode)."""
    cfg, layer, moe = full_layers(c)
    x = L.synth_x(cfg, T, seed=0, index=T)
    try:
        moe.set_act_precision(L.ACT_F16X2)
        two = run_and_check(cfg, layer, x, moe=moe)
        moe.set_act_precision(L.ACT_F16)
        one = run_and_check(cfg, layer, x, moe=moe)
    finally:
        moe.set_act_precision(L.ACT_F16)
    print(f"config {c} T={T}: F16 rel_l2={one['rel_l2']:.2e}, F16X2 rel_l2={two['rel_l2']:.2e}")
    assert two["rel_l2"] <= 2e-5
    assert one["rel_l2"] > 4 * two["rel_l2"]
