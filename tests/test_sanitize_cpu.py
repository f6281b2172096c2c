"""The reference ingest's sanitize_weights (rust/src/model/loader.rs:241-249:
NaN, +-Inf and |v| > 100 become 0, applied to every tensor load_layer and
load_special return, loader.rs:161 and :188), on both sides, without a GPU.

The oracle (lco_sanitize, the ingest inside lco_moe_forward) is pinned by the
rule's closed form: hand-built blocks whose decoded values are small exact
numbers (so the expected values are known without any decoder), with
outliers on both sides of the cut-off in every type.  The product's host
functions (lcmoe_dequantize, lcmoe_sanitize_blocks, used by lcmoe_create and
lcmoe_model_create at upload) are then checked against the pinned oracle.
"""
import numpy as np
import pytest

import lcoracle as O
import leafcutterllm_amd as L
from kquant_pack import pack_q4_k, pack_q6_k, pack_q8_0

NEXT_ABOVE_100 = np.nextafter(np.float32(100.0), np.float32(np.inf))


def u8(b: bytes) -> np.ndarray:
    return np.frombuffer(b, np.uint8).copy()


def rule(v: np.ndarray) -> np.ndarray:
    """loader.rs:241-249, written from the text of the rule."""
    v = np.asarray(v, np.float32)
    bad = np.isnan(v) | np.isinf(v) | (np.abs(v) > np.float32(100.0))
    return np.where(bad, np.float32(0.0), v).astype(np.float32)


def test_oracle_sanitize_closed_form():
    v = np.array([np.nan, np.inf, -np.inf, 100.0, -100.0, NEXT_ABOVE_100, -NEXT_ABOVE_100,
                  99.99, 0.0, -0.0, 1e-45, 3e38, -1e3, 1.0], np.float32)
    exp = np.array([0, 0, 0, 100, -100, 0, 0, 99.99, 0, -0.0, 1e-45, 0, 0, 1], np.float32)
    got = O.sanitize(v)
    assert np.array_equal(got, exp)
    # a zeroed value is +0; a kept -0 stays -0 (the rule only replaces)
    assert got[0].view(np.uint32) == 0 and got[5].view(np.uint32) == 0
    assert got[9].view(np.uint32) == 0x80000000


# Hand-built blocks: (type, bytes, count, exact decoded values before the rule,
# number of outliers Q4_K cannot zero in place)

def q8_blocks():
    q1 = [127, 100, -100, -101, -128, 0, 1, 50] + [3] * 24
    v1 = np.array(q1, np.float64) * 1.0
    q2 = [50, 51, -50, -51] + [0] * 28
    v2 = np.array(q2, np.float64) * 2.0
    q3 = [127, -127, 101] + [7] * 29
    v3 = np.array(q3, np.float64) * 0.5
    b = pack_q8_0(1.0, q1) + pack_q8_0(2.0, q2) + pack_q8_0(0.5, q3)
    return b, 96, np.concatenate([v1, v2, v3]), 0


def q4k_block():
    # d = 1, dmin = 0.5: v = sc * q - 0.5 * m, exact
    sc = [7, 63, 0, 8, 40, 63, 16, 1]
    m = [2, 0, 63, 63, 1, 63, 0, 1]
    q = np.zeros(256, int)
    q[0:32] = np.arange(32) % 16          # sub-block 0: 7q - 1, q = 15 -> 104
    q[32:64] = np.arange(32) % 3          # sub-block 1: 63q, q = 2 -> 126 (m = 0: zeroable)
    q[64:96] = 15                         # sub-block 2: -31.5
    q[96:128] = 15                        # sub-block 3: 8 * 15 - 31.5 = 88.5
    q[128:160] = np.arange(32) % 4        # sub-block 4: 40q - 0.5, q = 3 -> 119.5 (not zeroable)
    q[160:192] = np.arange(32) % 4        # sub-block 5: 63q - 31.5, q = 3 -> 157.5 (not zeroable)
    q[192:224] = np.arange(32) % 8        # sub-block 6: 16q, q = 7 -> 112 (zeroable)
    q[224:256] = 9                        # sub-block 7: 8.5
    sub = np.repeat(np.arange(8), 32)
    v = np.array(sc, np.float64)[sub] * q - 0.5 * np.array(m, np.float64)[sub]
    # q = 0 decodes to -dmin * m: zero only in sub-blocks with m = 0 (1 and 6)
    unz = int(np.sum((np.abs(v) > 100) & (np.array(m)[sub] != 0)))
    assert unz == 2 + 8 + 8  # sub-blocks 0, 4 and 5
    return pack_q4_k(1.0, 0.5, sc, m, q), 256, v, unz


def q6k_block():
    sc = [4, 1, 1, 1, 1, -4, 1, 1, 127, 1, 1, 1, 1, 1, 1, 1]
    q = np.zeros(256, int)
    q[0:16] = [25, 26, -25, -26, -32, 31, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9]   # 4q
    q[80:96] = [25, 31, -25, -26] + [1] * 12                                # -4q
    q[128:144] = [1, 0, -1] + [0] * 13                                       # 127q
    q[16:80] = 5
    v = np.array(sc, np.float64)[np.arange(256) // 16] * q
    return pack_q6_k(1.0, sc, q), 256, v, 0


def f32_tensor():
    v = np.array([np.nan, np.inf, -np.inf, 100.0, -100.0, NEXT_ABOVE_100, 5.0, -0.0], np.float32)
    return v.tobytes(), 8, v.astype(np.float64), 0


CASES = {
    "q8_0": (O.Q8_0, q8_blocks), "q4_k": (O.Q4_K, q4k_block), "q6_k": (O.Q6_K, q6k_block),
    "f32": (O.F32, f32_tensor),
}


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_ingest_sanitizes_every_type(name):
    qt, make = CASES[name]
    raw, n, v, _ = make()
    exp = rule(v)
    assert np.sum(exp != v.astype(np.float32)) >= 3 or name == "f32"  # outliers present
    got = O.ingest(qt, u8(raw), n)
    assert np.array_equal(got, exp), np.nonzero(got != exp)
    # the block decoders alone keep the outliers
    dec = O.dequant(qt, u8(raw), n)
    assert np.array_equal(np.isnan(dec), np.isnan(v.astype(np.float32)))
    assert np.array_equal(dec[~np.isnan(dec)], v.astype(np.float32)[~np.isnan(dec)])


def test_oracle_ingest_non_finite_scale_blocks():
    for qt, blk in ((O.Q8_0, pack_q8_0(np.inf, [1] * 32)), (O.Q8_0, pack_q8_0(np.nan, [0] * 32)),
                    (O.Q4_K, pack_q4_k(np.inf, 0.0, [1] * 8, [0] * 8, np.zeros(256, int))),
                    (O.Q4_K, pack_q4_k(0.5, np.nan, [1] * 8, [1] * 8, np.ones(256, int))),
                    (O.Q6_K, pack_q6_k(-np.inf, [1] * 16, np.zeros(256, int)))):
        n = 32 if qt == O.Q8_0 else 256
        assert not np.all(np.isfinite(O.dequant(qt, u8(blk), n)))
        assert np.array_equal(O.ingest(qt, u8(blk), n), np.zeros(n, np.float32))


def _random_blocks(qt, nblk, rng):
    """Random blocks whose scales make about a third of the elements exceed
    the cut-off, with some non-finite-scale blocks."""
    blocks = []
    for i in range(nblk):
        if qt == O.Q8_0:
            d = [1.0, 0.5, 0.9, np.inf, 0.01][i % 5]
            blocks.append(pack_q8_0(d, rng.integers(-128, 128, 32)))
        elif qt == O.Q4_K:
            d, dmin = [(1.0, 0.25), (0.3, 0.0), (2.0, 4.0), (np.nan, 1.0), (0.01, 0.01)][i % 5]
            blocks.append(pack_q4_k(d, dmin, rng.integers(0, 64, 8), rng.integers(0, 64, 8) * (i % 2),
                                    rng.integers(0, 16, 256)))
        else:
            d = [1.0, 0.25, np.inf, 0.02][i % 4]
            blocks.append(pack_q6_k(d, rng.integers(-128, 128, 16), rng.integers(-32, 32, 256)))
    return u8(b"".join(blocks))


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_K, O.Q6_K, O.F32])
def test_product_dequantize_equals_oracle(qt):
    rng = np.random.default_rng(qt)
    if qt == O.F32:
        v = (rng.standard_normal(4096) * 80).astype(np.float32)
        v[::97] = np.nan
        v[::101] = np.inf
        data, n = u8(v.tobytes()), 4096
    else:
        n = (32 if qt == O.Q8_0 else 256) * 40
        data = _random_blocks(qt, n // (32 if qt == O.Q8_0 else 256), rng)
    ref = O.ingest(qt, data, n)
    got = L.dequantize(qt, data, n, sanitize=True)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    raw = L.dequantize(qt, data, n, sanitize=False)
    dec = O.dequant(qt, data, n)
    assert np.array_equal(raw.view(np.uint32), dec.view(np.uint32))


@pytest.mark.parametrize("name", list(CASES))
def test_product_sanitize_blocks_writes_zero_codes(name):
    qt, make = CASES[name]
    raw, n, v, unz = make()
    exp = rule(v)
    fixed, zeroed, unzeroable = L.sanitize_blocks(qt, u8(raw), n)
    assert unzeroable == unz
    v32 = v.astype(np.float32)
    assert zeroed + unzeroable == int(np.sum(np.isnan(v32) | np.isinf(v32) | (np.abs(v32) > 100)))
    dec = O.dequant(qt, fixed, n)
    if unz:  # the outliers Q4_K cannot write as zero stay as they were
        left = np.abs(dec) > 100
        assert int(np.sum(left)) == unz
        assert np.array_equal(dec[~left], exp[~left])
    else:
        assert np.array_equal(dec, exp)  # -0 == +0 in value


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_product_sanitize_blocks_random(qt):
    rng = np.random.default_rng(100 + qt)
    bs = 32 if qt == O.Q8_0 else 256
    data = _random_blocks(qt, 60, rng)
    n = bs * 60
    ref = O.ingest(qt, data, n)
    fixed, zeroed, unz = L.sanitize_blocks(qt, data, n)
    dec = O.dequant(qt, fixed, n)
    if qt == O.Q4_K:
        assert unz > 0
        ok = np.abs(dec) <= 100
        assert int(np.sum(~ok)) == unz
        assert np.array_equal(dec[ok], ref[ok])
    else:
        assert unz == 0 and zeroed > 0
        assert np.array_equal(dec, ref)


def test_oracle_layer_sanitizes_router_and_bias():
    """lco_moe_forward ingests the router and the bias as load_layer ingests
    a layer tensor: NaN, inf and |v| > 100 entries act as 0."""
    cfg = L.configs.small_config("san", 256, 256, 8, 2, L.ROUTE_SOFTMAX, L.TYPE_Q8_0,
                                 L.TYPE_Q8_0)
    layer = L.synth_layer(cfg, seed=3)
    desc = O.Desc(**cfg.desc(4).as_dict())
    desc.has_bias = 1
    x = L.synth_x(cfg, 4, seed=3, index=0)
    bias = np.array([0.1, np.nan, 0.0, 150.0, -0.2, np.inf, 100.0, 0.0], np.float32)
    router = layer["router"].copy()
    router[3, 1] = np.nan
    router[10, 4] = -np.inf
    router[17, 6] = 101.0
    router[20, 2] = -100.0  # kept
    dirty = dict(layer, router=router, bias=bias)
    clean = dict(layer, router=rule(router), bias=rule(bias))
    a = O.moe_forward(desc, dirty, x)
    b = O.moe_forward(desc, clean, x)
    for k in ("y", "topk_idx", "topk_w"):
        assert np.array_equal(a[k], b[k]), k
    assert np.all(np.isfinite(a["y"]))
