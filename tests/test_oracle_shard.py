"""The oracle's shard-layout GEMM (lco_shard_matmul, restating
int8_gemm.rs q8_0_matmul / q4_0_matmul on x86), pinned by:
the reference's own tests (int8_gemm.rs:395-511: its test matrices against
dequantise-then-matmul within 1e-3), exact small-integer cases that fix the
operand order and the nibble order, and a float64 error bound."""
import numpy as np
import pytest

import lcoracle as O
from shard_pack import dequant, pack_q4, pack_q8, reference_test_matrices

Q8, Q4 = 8, O.Q4_0_SHARD


def _pack(qtype, scales, codes):
    return pack_q8(scales, codes) if qtype == Q8 else pack_q4(scales, codes)


@pytest.mark.parametrize("qtype", [Q8, Q4])
@pytest.mark.parametrize("m,k,n,a_fn", [
    (4, 8, 32, lambda i: i * 0.1),            # test_*_matmul_vs_dequant
    (8, 16, 64, lambda i: i * 0.01 - 0.5),    # test_*_matmul_large
])
def test_reference_tests(qtype, m, k, n, a_fn):
    a = np.array([a_fn(i) for i in range(m * k)], np.float32).reshape(m, k)
    scales, codes = reference_test_matrices(qtype, k, n)
    c = O.shard_matmul(qtype, a, _pack(qtype, scales, codes), k, n)
    expected = a.astype(np.float64) @ dequant(qtype, scales, codes).astype(np.float64)
    assert np.all(np.abs(c - expected) < 1e-3)


@pytest.mark.parametrize("qtype", [Q8, Q4])
def test_exact_integers_fix_order(qtype):
    """Scale 1 and small integers: every product and partial sum is exact, so
    C must equal the integer product; a transposed B, a wrong block stride or
    a swapped nibble order fails."""
    rng = np.random.default_rng(1)
    m, k, n = 3, 40, 96
    a = rng.integers(-9, 10, (m, k)).astype(np.float32)
    codes = (rng.integers(-100, 100, (k, n)) if qtype == Q8 else rng.integers(0, 16, (k, n)))
    scales = np.ones((k, n // 32), np.float32)
    c = O.shard_matmul(qtype, a, _pack(qtype, scales, codes), k, n)
    w = codes.astype(np.int64) - (8 if qtype == Q4 else 0)
    assert np.array_equal(c, (a.astype(np.int64) @ w).astype(np.float32))


@pytest.mark.parametrize("qtype", [Q8, Q4])
def test_float64_bound(qtype):
    rng = np.random.default_rng(2)
    m, k, n = 5, 300, 128
    a = rng.standard_normal((m, k)).astype(np.float32)
    codes = (rng.integers(-127, 128, (k, n)) if qtype == Q8 else rng.integers(0, 16, (k, n)))
    scales = rng.uniform(-0.02, 0.02, (k, n // 32)).astype(np.float32)
    c = O.shard_matmul(qtype, a, _pack(qtype, scales, codes), k, n)
    w = dequant(qtype, scales, codes).astype(np.float64)
    ref = a.astype(np.float64) @ w
    bound = (k + 1) * 2.0 ** -24 * (np.abs(a.astype(np.float64)) @ np.abs(w))
    assert np.all(np.abs(c - ref) <= bound + 1e-30)


def test_rejects_bad_shape():
    with pytest.raises(ValueError):
        O.shard_matmul(Q8, np.zeros((1, 4), np.float32), np.zeros(4 * 34, np.uint8), 4, 40)
