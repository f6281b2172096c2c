"""Pins the CPU oracle's building blocks (no GPU).

Each check is chosen so that a plausible mistake (wrong nibble half, wrong
scale index, FMA where the reference rounds twice, wrong tie rule) fails it;
expected values come from the reference's own tests, from numpy / float64,
from independent packers (tests/kquant_pack.py) or from closed forms.
"""
import math

import numpy as np
import pytest

import lcoracle as O
from kquant_pack import (expected_q4_k, expected_q6_k, pack_q4_k, pack_q6_k,
                         pack_q8_0)


def u8(b: bytes) -> np.ndarray:
    return np.frombuffer(b, np.uint8).copy()


# ---------------------------------------------------------------- f16 -------

def test_f16_to_f32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = O.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_vs_numpy():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # add ties, subnormal boundaries, overflow boundary
    extra = np.array([65504, 65519.99, 65520, 2.0**-24, 2.0**-25, 3 * 2.0**-26, 2.0**-14,
                      2.0**-14 - 2.0**-25, 1 + 2.0**-11, 1 + 3 * 2.0**-11, 0.0, -0.0,
                      np.inf, -np.inf], np.float32)
    x = np.concatenate([x, extra, -extra])
    ours = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(ours[nan].view(np.float16)))


# ---------------------------------------------------------- geometry -------

def test_block_geometry_reference_asserts():
    # quant.rs:314-335, gguf.rs:338-346
    assert O.tensor_size(O.Q4_K, 256) == 144
    assert O.tensor_size(O.Q6_K, 256) == 210
    assert O.tensor_size(O.Q8_0, 256) == 272
    assert O.tensor_size(O.F32, 100) == 400
    # row-straddling d_ff = 1408 tensor is sized on the flat count
    assert O.tensor_size(O.Q4_K, 2048 * 1408) == 2048 * 1408 // 256 * 144
    # per-expert bytes quoted for the Mixtral layer
    assert 3 * O.tensor_size(O.Q4_K, 4096 * 14336) == 99_090_432
    assert 3 * O.tensor_size(O.Q8_0, 1024 * 2816) == 9_191_424


# ---------------------------------------------------------- decoders -------

def test_zero_blocks_decode_to_zero():
    # kernels/mod.rs:235-251
    assert np.all(O.dequant(O.Q4_K, np.zeros(144, np.uint8), 256) == 0)
    assert np.all(O.dequant(O.Q6_K, np.zeros(210, np.uint8), 256) == 0)


def test_q8_0_reference_kat():
    # q8_0.rs:128-149: scale 0.5, qs[i] = i -> out[0] = 0, out[31] = 15.5
    blk = pack_q8_0(0.5, np.arange(32))
    out = O.dequant(O.Q8_0, u8(blk), 32)
    assert out[0] == 0.0 and out[31] == 15.5
    assert np.array_equal(out, np.arange(32, dtype=np.float32) * 0.5)
    neg = O.dequant(O.Q8_0, u8(pack_q8_0(-2.0, -np.arange(32) - 1)), 32)
    assert np.array_equal(neg, (np.arange(32, dtype=np.float32) + 1) * 2.0)


def test_scale_min_k4_all_subblocks():
    rng = np.random.default_rng(7)
    for _ in range(50):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        blk = pack_q4_k(1.0, 0.0, sc, m, np.zeros(256, int))
        for j in range(8):
            assert O.scale_min_k4(j, blk[4:16]) == (sc[j], m[j]), j


def test_q4_k_layout_kat():
    rng = np.random.default_rng(11)
    for trial in range(20):
        d = float(rng.choice([1.0, 0.5, 0.0078125, 1.5e-3]))
        dmin = float(rng.choice([0.0, 0.25, 3.0e-3]))
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        out = O.dequant(O.Q4_K, u8(pack_q4_k(d, dmin, sc, m, q)), 256)
        exp = expected_q4_k(d, dmin, sc, m, q)
        assert np.array_equal(out, exp), trial
    # positional KAT: d=1, dmin=0, sc=1: element e decodes to its own nibble
    q = np.array([(e * 7 + e // 32) % 16 for e in range(256)])
    out = O.dequant(O.Q4_K, u8(pack_q4_k(1.0, 0.0, [1] * 8, [0] * 8, q)), 256)
    assert np.array_equal(out, q.astype(np.float32))


def test_q6_k_layout_kat():
    rng = np.random.default_rng(12)
    for trial in range(20):
        d = float(rng.choice([1.0, 0.5, 1.2e-4]))
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(-32, 32, 256)
        out = O.dequant(O.Q6_K, u8(pack_q6_k(d, sc, q)), 256)
        assert np.array_equal(out, expected_q6_k(d, sc, q)), trial
    q = np.array([((e * 5) % 64) - 32 for e in range(256)])
    out = O.dequant(O.Q6_K, u8(pack_q6_k(1.0, [1] * 16, q)), 256)
    assert np.array_equal(out, q.astype(np.float32))


def test_multi_block_flat_decode_straddling_rows():
    # A [2, 1408] Q4_K tensor: 11 super-blocks, row 1 starts mid-block.
    rng = np.random.default_rng(3)
    blocks, exp = [], []
    for _ in range(11):
        sc, m, q = rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)
        blocks.append(pack_q4_k(0.01, 0.02, sc, m, q))
        exp.append(expected_q4_k(0.01, 0.02, sc, m, q))
    out = O.dequant(O.Q4_K, u8(b"".join(blocks)), 2 * 1408)
    assert np.array_equal(out, np.concatenate(exp))


def test_sanitize_and_scan():
    blk = bytearray(pack_q4_k(1.0, 0.0, [1] * 8, [0] * 8, np.zeros(256, int)))
    good = u8(bytes(blk) * 3)
    assert O.scan_blocks(O.Q4_K, good, 768) == 0
    bad = bytearray(bytes(blk) * 3)
    bad[144:146] = f16_inf = np.array([np.inf], np.float16).tobytes()
    bad[288 + 2:288 + 4] = np.array([np.nan], np.float16).tobytes()
    assert O.scan_blocks(O.Q4_K, u8(bytes(bad)), 768) == 2
    q6 = bytearray(pack_q6_k(1.0, [1] * 16, np.zeros(256, int)))
    q6[208:210] = np.array([2e4], np.float16).tobytes()
    assert O.scan_blocks(O.Q6_K, u8(bytes(q6)), 256) == 1
    # Q8_0: only the scale is checked, quants that look like an f16 inf are fine
    q8 = pack_q8_0(0.5, [0, -1] + [0] * 30)
    assert O.scan_blocks(O.Q8_0, u8(q8), 32) == 0


# ---------------------------------------------------------- encoders -------

def test_q8_0_reference_roundtrip():
    # q8_0.rs:151-166
    data = (np.arange(64, dtype=np.float32) - 32.0) * np.float32(0.1)
    qb = O.quantize(O.Q8_0, data)
    assert qb.size == 68
    out = O.dequant(O.Q8_0, qb, 64)
    assert np.max(np.abs(out - data)) < 0.1


def test_q8_0_encoder_kat_round_half_away():
    # max |v| = 63.5 -> scale 0.5 exactly; v / 0.5 = +-0.5 rounds away from 0
    v = np.zeros(32, np.float32)
    v[0], v[1], v[2], v[3] = 63.5, 0.25, -0.25, -63.5
    qb = O.quantize(O.Q8_0, v)
    assert qb[:2].tobytes() == np.array([0.5], np.float16).tobytes()
    q = qb[2:].view(np.int8)
    assert (q[0], q[1], q[2], q[3]) == (127, 1, -1, -127)
    assert np.all(q[4:] == 0)
    assert np.all(O.quantize(O.Q8_0, np.zeros(32, np.float32)) == 0)


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_encoder_roundtrip_error(qtype):
    x = O.synth_normal(5, 77, 0.02, 256 * 64)
    out = O.dequant(qtype, O.quantize(qtype, x), x.size)
    err = out - x
    rel = np.sqrt(np.mean(err**2)) / np.sqrt(np.mean(x**2))
    bound = {O.Q4_K: 0.09, O.Q6_K: 0.03, O.Q8_0: 0.01}[qtype]
    assert rel < bound, rel
    if qtype == O.Q4_K:  # per sub-block error <= one step (scale-rounding slack)
        blocks = O.quantize(qtype, x).reshape(-1, 144)
        for b in range(8):
            d = np.frombuffer(blocks[b, :2].tobytes(), np.float16)[0]
            for j in range(8):
                sc, _ = O.scale_min_k4(j, blocks[b, 4:16].tobytes())
                e = np.abs(err[256 * b + 32 * j: 256 * b + 32 * j + 32])
                assert e.max() <= float(d) * (sc + 8) + 1e-7


def test_q4_k_encoder_matches_independent_packer():
    # the encoder's bytes decode to q / sc / m values that the independent
    # packer re-packs to the identical block
    x = O.synth_normal(9, 3, 0.02, 256 * 4)
    qb = O.quantize(O.Q4_K, x).reshape(4, 144)
    for b in range(4):
        blk = qb[b].tobytes()
        d = float(np.frombuffer(blk[:2], np.float16)[0])
        dmin = float(np.frombuffer(blk[2:4], np.float16)[0])
        sm = [O.scale_min_k4(j, blk[4:16]) for j in range(8)]
        qs = np.frombuffer(blk[16:], np.uint8)
        q = np.empty(256, int)
        for jj in range(4):
            q[64 * jj: 64 * jj + 32] = qs[32 * jj: 32 * jj + 32] & 15
            q[64 * jj + 32: 64 * jj + 64] = qs[32 * jj: 32 * jj + 32] >> 4
        assert pack_q4_k(d, dmin, [s for s, _ in sm], [m for _, m in sm], q) == blk


# ------------------------------------------------------------ matmul -------

def ref_matmul_mul_add(a, b):
    """simd.rs:412-424 reference_matmul: sum += a*b, two roundings, f32."""
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            s = np.float32(0)
            for l in range(k):
                s = np.float32(s + np.float32(a[i, l] * b[l, j]))
            c[i, j] = s
    return c


def test_matmul_reference_kats():
    # simd.rs:430-455 (exact equality), tensor.rs:195-201
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[1, 0], [0, 1]], np.float32)
    assert np.array_equal(O.matmul(a, b), ref_matmul_mul_add(a, b))
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(1, 10, dtype=np.float32).reshape(3, 3)
    assert np.array_equal(O.matmul(a, b), ref_matmul_mul_add(a, b))
    # simd.rs:458-472 (|d| < 1e-4) and :486-504 (parallel == single)
    m, k, n = 16, 32, 24
    a = (np.arange(m * k, dtype=np.float32) * np.float32(0.01)).reshape(m, k)
    b = (np.arange(k * n, dtype=np.float32) * np.float32(0.01)).reshape(k, n)
    assert np.max(np.abs(O.matmul(a, b) - ref_matmul_mul_add(a, b))) < 1e-4
    m, k, n = 128, 256, 128
    a = (np.arange(m * k, dtype=np.float32) * np.float32(0.001)).reshape(m, k)
    b = (np.arange(k * n, dtype=np.float32) * np.float32(0.001)).reshape(k, n)
    c1, cp, cc = O.matmul(a, b, 1), O.matmul(a, b, 0), O.matmul(a, b, 4)
    assert np.array_equal(c1, cp) and np.array_equal(c1, cc)


def test_matmul_fma_lanes_and_unfused_tail():
    # columns 0..7 are fused (acc = fma(a, b, acc)), column 8 is a*b then +
    eps = np.float32(2.0**-12)
    a = np.array([[1.0, 1.0 + eps]], np.float32)
    b = np.vstack([-np.ones(9, np.float32), np.full(9, 1.0 + eps, np.float32)])
    c = O.matmul(a, b)[0]
    fused = np.float32(2.0**-11 + 2.0**-24)
    unfused = np.float32(2.0**-11)
    assert np.all(c[:8] == fused), c
    assert c[8] == unfused, c


def test_matmul_error_bound_vs_float64():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 700)).astype(np.float32)
    b = (rng.standard_normal((700, 37)) * 0.02).astype(np.float32)
    c = O.matmul(a, b).astype(np.float64)
    c64 = a.astype(np.float64) @ b.astype(np.float64)
    bound = 700 * 2.0**-24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(c - c64) <= bound)


# ------------------------------------------------------ silu / softmax -----

def test_silu_closed_form():
    v = np.linspace(-30, 30, 2001, dtype=np.float32)
    ours = np.array([O.silu(float(t)) for t in v], np.float32)
    ref = v.astype(np.float64) / (1.0 + np.exp(-v.astype(np.float64)))
    assert np.allclose(ours, ref, rtol=4e-7, atol=1e-30)
    assert O.silu(0.0) == 0.0


def test_rms_norm_reference_test_and_float64():
    """CpuBackend::rms_norm: the reference's own test (tensor.rs:204-209: finite
    output for [1, 2, 3]), a float64 closed form within a few ulp, exact
    results for constant rows, and the weight applied after the scale."""
    y = O.rms_norm(np.array([[1, 2, 3]], np.float32), np.ones(3, np.float32))
    assert np.all(np.isfinite(y))
    rng = np.random.default_rng(3)
    for d in (3, 8, 33, 256, 4096):
        x = rng.standard_normal((5, d)).astype(np.float32) * 3
        w = rng.standard_normal(d).astype(np.float32)
        y = O.rms_norm(x, w, 1e-5)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * w
        assert np.allclose(y, ref, rtol=4e-6, atol=1e-30), d
    # a constant row c: mean_sq = c^2 exactly (powers of two), scale = 1/sqrt(c^2 + eps)
    for c in (0.5, 2.0, 8.0):
        x = np.full((1, 64), c, np.float32)
        y = O.rms_norm(x, np.ones(64, np.float32), 0.0)
        assert np.all(y == np.float32(1.0)), c
    # scale before weight: (x * s) * w, two roundings
    x = np.array([[3.0, 4.0, 0.0, 0.0]], np.float32)
    w = np.array([1.1, 0.7, 1.0, 1.0], np.float32)
    s = np.float32(1.0) / np.sqrt(np.float32(25.0 / 4.0) + np.float32(1e-5))
    assert np.array_equal(O.rms_norm(x, w, 1e-5)[0, :2],
                          (np.float32(x[0, :2] * s) * w[:2]).astype(np.float32))


def _rms_norm_four_lanes(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """CpuBackend::rms_norm (cpu.rs:49-60) over x86 simd_sum_sq
    (kernels/simd.rs:390-409), written out in numpy float32: lane l sums
    round(v*v) of elements l, l+4, ... as acc = round(v*v) + acc (product
    then add, no FMA); the lanes add as ((a0 + a1) + a2) + a3; the tail past
    the last group of four adds one square at a time; mean = sum / n,
    scale = 1 / sqrt(mean + eps), out = (x * scale) * w."""
    x = np.asarray(x, np.float32)
    T, n = x.shape
    m = n // 4 * 4
    acc = np.zeros((T, 4), np.float32)
    for i in range(0, m, 4):
        v = x[:, i:i + 4]
        acc = (v * v) + acc
    s = ((acc[:, 0] + acc[:, 1]) + acc[:, 2]) + acc[:, 3]
    for r in range(m, n):
        s = s + x[:, r] * x[:, r]
    mean = s / np.float32(n)
    scale = np.float32(1.0) / np.sqrt(mean + np.float32(eps))
    return (x * scale[:, None]) * np.asarray(w, np.float32)


def _rms_norm_sequential(x, w, eps):
    """The same with one sequential sum: the order a four-lane oracle must not use."""
    x = np.asarray(x, np.float32)
    s = np.zeros(x.shape[0], np.float32)
    for r in range(x.shape[1]):
        s = s + x[:, r] * x[:, r]
    scale = np.float32(1.0) / np.sqrt(s / np.float32(x.shape[1]) + np.float32(eps))
    return (x * scale[:, None]) * np.asarray(w, np.float32)


def test_rms_norm_four_lane_order_bit_exact():
    """lco_rms_norm reproduces the reference's four-lane sum-of-squares order
    bit for bit, on rows with spread magnitudes where a sequential sum (or a
    pairwise / float64 one) rounds differently."""
    rng = np.random.default_rng(11)
    for d in (4, 7, 64, 130, 1024, 4096):
        T = 200
        x = (rng.standard_normal((T, d)) * 10.0 ** rng.uniform(-3, 3, (T, d))).astype(np.float32)
        w = rng.standard_normal(d).astype(np.float32)
        ours = O.rms_norm(x, w, 1e-5)
        lanes = _rms_norm_four_lanes(x, w, 1e-5)
        assert np.array_equal(ours.view(np.uint32), lanes.view(np.uint32)), d
        if d >= 64:  # the order matters on these rows: a sequential oracle fails
            seq = _rms_norm_sequential(x, w, 1e-5)
            differ = np.any(seq.view(np.uint32) != lanes.view(np.uint32), axis=1)
            assert differ.sum() >= T // 10, (d, differ.sum())


def test_softmax_kat_and_closed_form():
    y = O.softmax(np.array([1.0, 2.0, 3.0], np.float32))  # tensor.rs:211-217
    assert abs(float(np.sum(y)) - 1.0) < 1e-5
    rng = np.random.default_rng(2)
    x = rng.standard_normal(60).astype(np.float32) * 3
    ref = np.exp(x.astype(np.float64) - x.max()) / np.exp(x.astype(np.float64) - x.max()).sum()
    assert np.allclose(O.softmax(x), ref, rtol=2e-6)


def _ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


def test_expf_cw_within_2ulp_of_float64():
    x = np.concatenate([np.linspace(-103.9, 88.7, 200001, dtype=np.float32),
                        np.linspace(-1, 1, 20001, dtype=np.float32)])
    ours = O.expf_cw(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    normal = ref >= np.float32(2.0**-126)
    assert _ulp_diff(ours[normal], ref[normal]).max() <= 2
    # subnormal results: absolute error within 2 subnormal ulps
    assert np.max(np.abs(ours[~normal].astype(np.float64) - ref[~normal]) / 2.0**-149) <= 2
    assert O.expf_cw(np.array([0.0]))[0] == 1.0
    sp = O.expf_cw(np.array([np.inf, -np.inf, 100.0, -200.0], np.float32))
    assert sp[0] == np.inf and sp[1] == 0.0 and sp[2] == np.inf and sp[3] == 0.0
    assert np.isnan(O.expf_cw(np.array([np.nan], np.float32))[0])


def test_sigmoid_cw_closed_form():
    x = np.linspace(-20, 20, 40001, dtype=np.float32)
    s = O.sigmoid_cw(x)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(s - ref) / ref) < 5e-7
    assert np.all(np.diff(s) >= 0)


# ------------------------------------------------------------ synth ---------

def test_synth_normal_is_counter_based_and_normal():
    a = O.synth_normal(42, 5, 1.0, 200001)
    b = O.synth_normal(42, 5, 1.0, 1000)
    assert np.array_equal(a[:1000], b)
    assert not np.array_equal(a[:1000], O.synth_normal(42, 6, 1.0, 1000))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    s = O.synth_normal(42, 5, 0.02, 1000)
    assert np.allclose(s, (a[:1000].astype(np.float64) * 0.02).astype(np.float32), rtol=1e-6)
